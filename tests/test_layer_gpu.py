"""One GDN layer end to end (braid_amd.mixer.GDNMixerLayer) at the Qwen3.5
shape (32 value heads, 16 key groups) against a CPU restatement of the
reference layer built only from the oracle.

The restatement follows braid/model/gdn.py:107-167 (decode), :171-226 and
:273-291 (prefill) and :373-387 (readout): causal conv with SiLU, the Q | K | V
split of the conv output (braid/config.py:34-44: q = channels [0, G*SS),
k = [G*SS, 2*G*SS), v = the rest, each unflattened per head), the in-kernel
gate formulas, the recurrence, the gated RMSNorm and the per-tensor FP8
quantization of its result. A wrong split order, stride, head map or readout
reshape in the layer glue moves whole heads and fails here; errors shared by
the layer's decode and prefill paths, which test_mixer_graph_gpu compares
with each other, cannot hide from it. (Reference counterparts:
tests/test_copy_kill.py:167, tests/test_gdn_prefill_kernel.py:211,
tests/test_gdn_raw_gates.py:261.)

Bars: conv windows bitwise; fp16 states within one ulp after one token, and
within the free-running bound after a chunk; `core` within two bf16 ulps of
its (token, head) unit's rms, with >= 90% of elements bitwise (the kernel and
the oracle sum the recurrence in different orders, so y differs by a few
ulps of its scale, and an element of y near zero carries that as a large
error relative to itself; the RMSNorm then maps it onto `core`); FP8 codes and
scale bitwise equal to the quantization of the layer's own `core`, and the
scale within one bf16 ulp of the restatement's. A glue error (split order,
stride, head map, readout reshape) moves whole units by O(1) of their rms.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from braid_amd.cache import GDNCache
from braid_amd.config import GDNConfig
from braid_amd.mixer import GDNMixerLayer
from gpu_helpers import DEV, act_np, assert_free_running_close, gen, ulp16

pytestmark = pytest.mark.gpu
G = GDNConfig(n_heads=32, head_dim=128, state_size=128, n_groups=16, n_gdn_layers=1)
ACT = torch.bfloat16
EPS = 1e-6


def _weights(seed):
    C = G.conv_channels
    return {"conv1d": (torch.randn(C, 4, generator=gen(seed), device=DEV) * 0.3).to(ACT),
            "conv1d_bias": torch.randn(C, generator=gen(seed + 1), device=DEV) * 0.1,
            "A": -torch.exp(torch.rand(G.n_heads, generator=gen(seed + 2), device=DEV) * 2),
            "dt_bias": torch.rand(G.n_heads, generator=gen(seed + 3), device=DEV) * 2 - 1,
            "norm": 1 + 0.3 * torch.randn(G.head_dim, generator=gen(seed + 4), device=DEV)}


def _cache(n_slots, seed):
    cache = GDNCache.allocate(G, n_slots, DEV, torch.float16)
    lyr = cache.layers[0]
    lyr.state.copy_(torch.randn(lyr.state.shape, generator=gen(seed), device=DEV) * 0.05)
    lyr.conv.copy_(torch.randn(lyr.conv.shape, generator=gen(seed + 1), device=DEV))
    return cache


def _inputs(B, T, seed):
    return (torch.randn(B, T, G.conv_channels, generator=gen(seed), device=DEV).to(ACT),
            (torch.randn(B, T, G.inner_size, generator=gen(seed + 1), device=DEV) * 2).to(ACT),
            torch.randn(B, T, G.n_heads, generator=gen(seed + 2), device=DEV).to(ACT),
            torch.randn(B, T, G.n_heads, generator=gen(seed + 3), device=DEV).to(ACT))


def _split(conv_out):
    """[..., C] -> q, k [..., G, SS], v [..., H, HD] (config.py:34-44)."""
    kd = G.n_groups * G.state_size
    q = conv_out[..., :kd].reshape(*conv_out.shape[:-1], G.n_groups, G.state_size)
    k = conv_out[..., kd:2 * kd].reshape(*conv_out.shape[:-1], G.n_groups, G.state_size)
    v = conv_out[..., 2 * kd:].reshape(*conv_out.shape[:-1], G.n_heads, G.head_dim)
    return q, k, v


def _restated_layer(w, state, conv, slots, qkv, z, a, b, seq_lens=None):
    """The reference layer on the oracle. state / conv: numpy pools (fp16 and
    fp32), updated in place. Returns core in bf16 storage [B, T, H*HD]."""
    B, T, _ = qkv.shape
    x = qkv.float().cpu().numpy()
    wc = w["conv1d"].float().cpu().numpy()
    bc = w["conv1d_bias"].cpu().numpy()
    lens = None if seq_lens is None else np.asarray(seq_lens, np.int32)
    if T == 1 and lens is None:
        conv_out = oracle.conv1d_decode(conv, slots, x[:, 0], wc, bc)[:, None]
    else:
        conv_out = oracle.conv1d_prefill(conv, slots, x, wc, bc, lens)
    q, k, v = _split(conv_out)
    alpha, beta = oracle.gdn_gates(act_np(a), act_np(b), w["A"].cpu().numpy(),
                                   w["dt_bias"].cpu().numpy(), "bf16", seq_lens=lens)
    y = oracle.gdn_prefill(state, slots, q, k, v, alpha, beta, "f16")
    zb = act_np(z).reshape(B, T, G.n_heads, G.head_dim)
    core = oracle.gated_rmsnorm(y, zb, w["norm"].cpu().numpy(), EPS, "bf16")
    return core.reshape(B, T, G.inner_size)


def _check_core(got_bits, ref_bits, what):
    g = oracle.widen(got_bits, "bf16").reshape(-1, G.head_dim).astype(np.float64)
    r = oracle.widen(ref_bits, "bf16").reshape(-1, G.head_dim).astype(np.float64)
    rms = np.sqrt(np.mean(r * r, axis=1, keepdims=True)) + 1e-30
    err = float((np.abs(g - r) / rms).max())
    same = float((got_bits == ref_bits).mean())
    print(f"  {what}: core max error {err:.2e} of its unit's rms (bar 2^-6 = 1.56e-02), "
          f"{100 * same:.2f}% bitwise", flush=True)
    assert err <= 2.0 ** -6, (what, err)
    assert same >= 0.90, (what, same)


def _check_layer_out(out, core_ref, live, what):
    core, xq, sx = out
    got = core.view(torch.uint16).cpu().numpy()
    _check_core(got[live], core_ref[live], what)
    # the FP8 quantization is an exact function of the layer's own core ...
    qo, so = oracle.quantize_act(core.float().cpu().numpy())
    assert sx.item() == float(so)
    assert np.array_equal(xq.view(torch.uint8).cpu().numpy(), qo)
    # ... and its scale is the restatement's to within the readout's rounding
    _, so_ref = oracle.quantize_act(oracle.widen(core_ref, "bf16"))
    assert abs(sx.item() - float(so_ref)) <= float(so_ref) * 2 ** -7


def test_layer_decode_matches_the_restated_reference():
    w = _weights(1)
    layer = GDNMixerLayer(G, w, eps=EPS, fp8_out=True)
    assert layer.fused_decode  # 2 value heads per key group: the fused launch
    cache = _cache(8, seed=2)
    slots = [5, 2, 7, 0]
    view = cache.select(slots)
    state = cache.layers[0].state.cpu().numpy().copy()
    conv = cache.layers[0].conv.cpu().numpy().copy()
    for step, seed in enumerate((10, 20, 30)):
        qkv, z, a, b = _inputs(len(slots), 1, seed)
        out = layer.decode(qkv, z, a, b, view.layers[0], view.slots_i32)
        torch.cuda.synchronize()
        core_ref = _restated_layer(w, state, conv, slots, qkv, z, a, b)
        _check_layer_out(out, core_ref, np.s_[:], f"decode step {step}")
        got_conv = cache.layers[0].conv.cpu().numpy()
        assert np.array_equal(got_conv.view(np.uint32), conv.view(np.uint32)), step
        got_state = cache.layers[0].state.cpu().numpy()
        d = ulp16(got_state[slots], state[slots])
        print(f"  decode step {step}: state within {int(d.max())} fp16 ulp", flush=True)
        assert d.max() <= 1
        # teacher forcing: the next step starts from the kernel's state
        state = got_state.copy()
    untouched = [1, 3, 4, 6]
    assert np.array_equal(cache.layers[0].state.cpu().numpy()[untouched], state[untouched])


def test_layer_prefill_matches_the_restated_reference():
    w = _weights(3)
    layer = GDNMixerLayer(G, w, eps=EPS, fp8_out=True)
    cache = _cache(6, seed=4)
    slots = [4, 1, 3]
    lens = [24, 9, 0]
    T = max(lens)
    view = cache.select(slots)
    state = cache.layers[0].state.cpu().numpy().copy()
    conv = cache.layers[0].conv.cpu().numpy().copy()
    qkv, z, a, b = _inputs(len(slots), T, 40)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = layer.prefill(qkv, z, a, b, view.layers[0], view.slots_i32, seq)
    torch.cuda.synchronize()
    core_ref = _restated_layer(w, state, conv, slots, qkv, z, a, b, seq_lens=lens)
    live = np.zeros((len(slots), T), bool)
    for r, n in enumerate(lens):
        live[r, :n] = True
    _check_layer_out(out, core_ref, live, "prefill")
    assert bool((out[0][~torch.from_numpy(live).to(DEV)] == 0).all()), "pad readouts not 0"
    got_conv = cache.layers[0].conv.cpu().numpy()
    assert np.array_equal(got_conv.view(np.uint32), conv.view(np.uint32))
    got_state = cache.layers[0].state.cpu().numpy()
    assert_free_running_close(got_state[slots], state[slots], "f16")
