"""The GDN layer glue (braid_amd.mixer) and the per-bucket graph decoder
(braid_amd.graph) on the GPU.

* prefill through the stack (conv prefill -> chunk scan -> readout) equals the
  decode step applied token by token: conv windows bitwise, states bitwise up
  to the sign of zero (a pad step computes 1*S + 0), and
  every live token's readout `core` bitwise (the readout is per token; only
  the FP8 scale spans the call);
* a graph-replayed bucket equals the eager step on the same rows, bitwise:
  states, windows, core, FP8 codes and scale, with padded rows pointed at a
  scratch slot (their zeroed gate makes their readout 0, so the scale is the
  live rows' own);
* capture leaves the pool as it found it; a new slot assignment replays the
  same graph; a padded batch without scratch slots is refused.
(reference: braid/model/gdn.py:107-167, :273-291, :373-387;
braid/model/graph.py:51-192; tests/test_slot_indirection.py)
"""
from __future__ import annotations

import pytest
import torch

from braid_amd.cache import GDNCache
from braid_amd.config import GDNConfig
from braid_amd.graph import GraphedDecoder
from braid_amd.mixer import GDNMixerLayer, mixer_decode_step
from gpu_helpers import DEV, gen

pytestmark = pytest.mark.gpu
G = GDNConfig(n_heads=8, head_dim=128, state_size=128, n_groups=4, n_gdn_layers=2)
ACT = torch.bfloat16


def _layers(n, fp8_out=True, seed=0):
    out = []
    for i in range(n):
        s = seed + 10 * i
        C = G.conv_channels
        w = {"conv1d": (torch.randn(C, 4, generator=gen(s), device=DEV) * 0.3).to(ACT),
             "conv1d_bias": torch.randn(C, generator=gen(s + 1), device=DEV) * 0.1,
             "A": -torch.exp(torch.rand(G.n_heads, generator=gen(s + 2), device=DEV) * 2),
             "dt_bias": torch.rand(G.n_heads, generator=gen(s + 3), device=DEV) * 2 - 1,
             "norm": 1 + 0.3 * torch.randn(G.head_dim, generator=gen(s + 4), device=DEV)}
        out.append(GDNMixerLayer(G, w, eps=1e-6, fp8_out=fp8_out))
    return out


def _cache(slots, state_dtype=torch.float16, seed=5):
    cache = GDNCache.allocate(G, slots, DEV, state_dtype)
    for i, lyr in enumerate(cache.layers):
        lyr.state.copy_(torch.randn(lyr.state.shape, generator=gen(seed + i), device=DEV) * 0.05)
        lyr.conv.copy_(torch.randn(lyr.conv.shape, generator=gen(seed + 50 + i), device=DEV))
    return cache


def _inputs(L, B, T, seed):
    return {"qkv": [torch.randn(B, T, G.conv_channels, generator=gen(seed + i), device=DEV)
                    .to(ACT) for i in range(L)],
            "z": [(torch.randn(B, T, G.inner_size, generator=gen(seed + 20 + i), device=DEV) * 2)
                  .to(ACT) for i in range(L)],
            "a": [torch.randn(B, T, G.n_heads, generator=gen(seed + 40 + i), device=DEV).to(ACT)
                  for i in range(L)],
            "b": [torch.randn(B, T, G.n_heads, generator=gen(seed + 60 + i), device=DEV).to(ACT)
                  for i in range(L)]}


def _bits(t):
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


def _same(a, b):
    if isinstance(a, torch.Tensor):
        return torch.equal(_bits(a), _bits(b))
    return all(_same(x, y) for x, y in zip(a, b))


def test_prefill_stack_equals_decode_token_by_token():
    L, lens, T = 2, [9, 4, 0, 6], 9
    layers = _layers(L, fp8_out=False)
    slots = [3, 0, 6, 5]
    x = _inputs(L, len(lens), T, seed=100)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)

    pre = _cache(8)
    view = pre.select(slots)
    core_p = [lyr.prefill(x["qkv"][i], x["z"][i], x["a"][i], x["b"][i], view.layers[i],
                          view.slots_i32, seq) for i, lyr in enumerate(layers)]

    dec = _cache(8)
    for r, n in enumerate(lens):
        v1 = dec.select([slots[r]])
        for t in range(n):
            for i, lyr in enumerate(layers):
                core = lyr.decode(x["qkv"][i][r:r + 1, t:t + 1], x["z"][i][r:r + 1, t:t + 1],
                                  x["a"][i][r:r + 1, t:t + 1], x["b"][i][r:r + 1, t:t + 1],
                                  v1.layers[i], v1.slots_i32)
                assert torch.equal(core[0, 0].view(torch.int16),
                                   core_p[i][r, t].view(torch.int16)), (r, t, i)
    torch.cuda.synchronize()
    for a, b in zip(pre.layers, dec.layers):
        assert torch.equal(a.conv.view(torch.int32), b.conv.view(torch.int32))
        # value-equal; bitwise except that a pad step (1*S + 0) may turn a
        # stored -0 into +0, as the reference's arithmetic does
        assert torch.equal(a.state, b.state)
        diff = a.state.view(torch.int16) != b.state.view(torch.int16)
        assert bool((a.state[diff] == 0).all())


def _make_inputs(L):
    def make(size):
        return {"qkv": [torch.zeros(size, 1, G.conv_channels, device=DEV, dtype=ACT)
                        for _ in range(L)],
                "z": [torch.zeros(size, 1, G.inner_size, device=DEV, dtype=ACT) for _ in range(L)],
                "a": [torch.zeros(size, 1, G.n_heads, device=DEV, dtype=ACT) for _ in range(L)],
                "b": [torch.zeros(size, 1, G.n_heads, device=DEV, dtype=ACT) for _ in range(L)]}
    return make


def test_graph_buckets_equal_the_eager_step():
    L, S, scratch = 2, 16, 15
    layers = _layers(L)
    step = mixer_decode_step(layers)
    cache = _cache(S)
    s0 = cache.snapshot()
    gd = GraphedDecoder(step, cache, _make_inputs(L), buckets=(1, 2, 4, 8), warmup=2)
    torch.cuda.synchronize()
    assert gd.sizes == (1, 2, 4, 8)
    assert _same(cache.snapshot(), s0), "capture changed the pool"

    for label, rows, seed in (("pad 3->4", [5, 9, 2], 300), ("reassign 2", [7, 5], 400),
                              ("pad 5->8", [0, 11, 3, 8, 14], 500)):
        x = _inputs(L, len(rows), 1, seed)
        slots = torch.tensor(rows, dtype=torch.int64, device=DEV)
        start = cache.snapshot()
        out_g = gd.step(x, slots, pad_slots=torch.full((8,), scratch, device=DEV))
        torch.cuda.synchronize()
        after_g = cache.snapshot()
        cache.restore(start)
        out_e = step(x, cache.select(rows))
        torch.cuda.synchronize()
        after_e = cache.snapshot()
        for i in range(L):
            core_g, q_g, s_g = out_g[i]
            core_e, q_e, s_e = out_e[i]
            assert core_g.shape == core_e.shape, label
            assert _same(core_g, core_e), (label, i, "core")
            assert _same(s_g, s_e), (label, i, "scale", s_g.item(), s_e.item())
            assert _same(q_g, q_e), (label, i, "fp8")
        live = [r for r in range(S) if r != scratch]
        for a, b in zip(after_g[1:], after_e[1:]):
            assert _same(a[live], b[live]), label
        cache.restore(after_g)


def test_padded_batch_needs_scratch_slots():
    L = 1
    cache = _cache(8)
    gd = GraphedDecoder(mixer_decode_step(_layers(L)), cache, _make_inputs(L), buckets=(4,),
                        warmup=1)
    x = _inputs(L, 3, 1, seed=7)
    with pytest.raises(ValueError, match="pass pad_slots"):
        gd.step(x, torch.tensor([1, 2, 3], device=DEV))
    with pytest.raises(ValueError, match="exceeds the largest bucket"):
        gd.step(_inputs(L, 5, 1, seed=8), torch.arange(5, device=DEV))
    # a replay skips the kernels' eager checks, so step() makes them
    scratch = torch.tensor([7], device=DEV)
    with pytest.raises(ValueError, match="duplicate slot 1"):
        gd.step(x, torch.tensor([1, 2, 1], device=DEV), pad_slots=scratch)
    with pytest.raises(ValueError, match="out of range"):
        gd.step(x, torch.tensor([1, 2, 8], device=DEV), pad_slots=scratch)
    with pytest.raises(ValueError, match="also a live slot"):
        gd.step(x, torch.tensor([1, 2, 7], device=DEV), pad_slots=scratch)
