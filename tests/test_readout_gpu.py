"""Gated RMSNorm readout (+ out_proj input FP8 quant) on the GPU.

The readout is braid/model/gdn.py:373-387 with braid/model/norm.py:48-71 and,
for an FP8 out_proj, quantize_act (braid/model/quant.py:209-229) on the
result. Its fp32 reduction order differs from torch's rms_norm kernel, so
`core` is gated by tolerance (refmath.READOUT_ULPS): against the oracle and
against torch's own spelling on this device, >= 99.5% of 16-bit elements
bit-identical and none more than 3 ulp apart; fp32 activations within 8 ulp.
The FP8 codes and scale are bit-exact functions of `core`, checked bitwise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import DEV, gen
from refmath import (ACT_DTYPES, READOUT_ULPS, act_storage, act_ulps, check_readout,
                     torch_gated_readout)

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _inputs(N, H, act, seed, y_scale=0.05):
    y = torch.randn(N, H, 128, generator=gen(seed), device=DEV) * y_scale
    z = (torch.randn(N, H * 128, generator=gen(seed + 1), device=DEV) * 2).to(ACT_DTYPES[act])
    gamma = 1.0 + 0.3 * torch.randn(128, generator=gen(seed + 2), device=DEV)
    return y, z, gamma


@pytest.mark.parametrize("act", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("N", [1, 64, 4073], ids=["tok1", "decode64", "prefill4073"])
def test_core_matches_oracle_and_torch(kern, act, N):
    y, z, gamma = _inputs(N, 32, act, seed=N)
    core, q, scale = kern.gated_rmsnorm(y, z, gamma, EPS)
    assert core.dtype == ACT_DTYPES[act] and tuple(core.shape) == tuple(z.shape)
    ref_t = torch_gated_readout(y.reshape(N, 32, 128), z.reshape(N, 32, 128), gamma, EPS,
                                ACT_DTYPES[act]).reshape(z.shape)
    check_readout(act_storage(core, act), act_storage(ref_t, act), act, "torch")
    ref_o = oracle.gated_rmsnorm(y.cpu().numpy(), act_storage(z, act).reshape(N, 32, 128),
                                 gamma.cpu().numpy(), EPS, act).reshape(N, 32 * 128)
    check_readout(act_storage(core, act), ref_o, act, "oracle")


@pytest.mark.parametrize("act", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("N", [1, 64, 4073], ids=["tok1", "decode64", "prefill4073"])
def test_quant_is_quantize_act_of_core_bitwise(kern, act, N):
    y, z, gamma = _inputs(N, 32, act, seed=100 + N)
    core, q, scale = kern.gated_rmsnorm(y, z, gamma, EPS)
    q2, s2 = kern.quantize_act(core)
    assert q.dtype == torch.float8_e4m3fn and tuple(scale.shape) == (1, 1)
    assert torch.equal(scale, s2)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    qo, so = oracle.quantize_act(core.float().cpu().numpy())
    assert scale.item() == float(so)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qo)


def test_norm_only_and_y_in_act_dtype(kern):
    y, z, gamma = _inputs(64, 32, "bf16", seed=7)
    core, _, _ = kern.gated_rmsnorm(y, z, gamma, EPS)
    alone = kern.gated_rmsnorm(y, z, gamma, EPS, quantize=False)
    assert torch.equal(alone.view(torch.uint16), core.view(torch.uint16))
    # The reference casts y to the act dtype first, so a bf16 y gives the same bits.
    pre = kern.gated_rmsnorm(y.bfloat16(), z, gamma, EPS, quantize=False)
    assert torch.equal(pre.view(torch.uint16), core.view(torch.uint16))


@pytest.mark.parametrize("units", [1, 3, 7, 9, 8191, 8193])
def test_ragged_unit_counts(kern, units):
    """Unit counts that leave a half-wave, a wave and a block partly empty,
    and that wrap the 1024-block grid-stride loop."""
    y = torch.randn(units, 128, generator=gen(units), device=DEV)
    z = torch.randn(units, 128, generator=gen(units + 1), device=DEV).bfloat16()
    gamma = torch.ones(128, device=DEV)
    core, q, scale = kern.gated_rmsnorm(y, z, gamma, EPS)
    ref = oracle.gated_rmsnorm(y.cpu().numpy(), act_storage(z, "bf16"), gamma.cpu().numpy(),
                               EPS, "bf16")
    assert act_ulps(act_storage(core, "bf16"), ref, "bf16").max() <= READOUT_ULPS["bf16"]
    qo, so = oracle.quantize_act(core.float().cpu().numpy())
    assert scale.item() == float(so)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qo)


def test_nan_propagates_to_the_scale(kern):
    y, z, gamma = _inputs(8, 32, "bf16", seed=9)
    y[3, 5, 17] = float("nan")
    core, q, scale = kern.gated_rmsnorm(y, z, gamma, EPS)
    assert torch.isnan(scale).all()
    assert torch.isnan(core[3, 5 * 128:6 * 128].float()).all()
    assert (q.view(torch.uint8) & 0x7F == 0x7F).all()


def test_zero_gate_and_empty_input(kern):
    y, z, gamma = _inputs(4, 32, "bf16", seed=11)
    core, q, scale = kern.gated_rmsnorm(y, torch.zeros_like(z), gamma, EPS)
    assert (core.float() == 0).all() and scale.item() == np.float32(1e-12)
    assert ((q.view(torch.uint8) & 0x7F) == 0).all()  # +0 or -0, as the sign of xf
    empty = kern.gated_rmsnorm(torch.empty(0, 32, 128, device=DEV),
                               torch.empty(0, 4096, device=DEV, dtype=torch.bfloat16),
                               gamma, EPS, quantize=False)
    assert empty.numel() == 0
    with pytest.raises(RuntimeError, match="must not be empty"):
        kern.gated_rmsnorm(torch.empty(0, 32, 128, device=DEV),
                           torch.empty(0, 4096, device=DEV, dtype=torch.bfloat16), gamma, EPS)


def test_argument_checks(kern):
    y, z, gamma = _inputs(4, 32, "bf16", seed=12)
    with pytest.raises(RuntimeError, match="head_dim=128"):
        kern.gated_rmsnorm(y.reshape(4, 64, 64), z, gamma[:64].contiguous(), EPS)
    with pytest.raises(RuntimeError, match="same number"):
        kern.gated_rmsnorm(y[:2], z, gamma, EPS)
    with pytest.raises(RuntimeError, match="fp32 or z's dtype"):
        kern.gated_rmsnorm(y.half(), z, gamma, EPS)


def test_silu_gate_is_torchs_spelling_bit_for_bit(kern):
    """With fp32 activations, y = 1, gamma = 1 and eps = 0 the norm is exactly
    1, so core = silu(z) as the kernel computes it: z / (1 + exp(-z)) with
    an IEEE division (braid/model/norm.py:67-71 through F.silu). Every finite
    bf16 value as z, 4M random fp32 bit patterns and wide normals must equal
    torch's spelling on the same device bit for bit (NaN for NaN)."""
    every = torch.arange(0, 1 << 16, device=DEV, dtype=torch.int32).to(torch.int16)
    every = every.view(torch.bfloat16).float()
    every = every[torch.isfinite(every)]
    g = gen(41)
    bits = torch.randint(-2 ** 31, 2 ** 31 - 1, (1 << 22,), generator=g, device=DEV,
                         dtype=torch.int32).view(torch.float32)
    z = torch.cat([every, bits[torch.isfinite(bits)],
                   torch.randn(1 << 20, generator=g, device=DEV) * 30])
    n = z.numel() - z.numel() % 128
    z = z[:n].contiguous()
    units = n // 128
    core = kern.gated_rmsnorm(torch.ones(units, 1, 128, device=DEV), z.view(units, 128),
                              torch.ones(128, device=DEV), 0.0, quantize=False)
    core = (core[0] if isinstance(core, (tuple, list)) else core).reshape(-1)
    ref = z / (1 + torch.exp(-z))
    same = (core.view(torch.int32) == ref.view(torch.int32)) | (core.isnan() & ref.isnan())
    bad = (~same).nonzero().flatten()[:5]
    assert bad.numel() == 0, (z[bad].tolist(), core[bad].tolist(), ref[bad].tolist())
