"""The fused conv1d + GDN decode launch (braid_gdn_conv_decode_raw) against
the two kernels it fuses, run back to back as the reference's decode does
(braid/model/gdn.py:131-160: conv1d_decode, then gdn_decode_raw on the
split/unflatten views of the conv output). Outputs, states and conv windows
must be bit-identical, and slots outside the batch untouched."""
from __future__ import annotations

import pytest
import torch

from gpu_helpers import DEV, gen, raw_gates

pytestmark = pytest.mark.gpu


def _setup(B, H, G, S, pool_dt, x_dt, seed, with_bias=True):
    C = 2 * G * 128 + H * 128
    pool = (torch.randn(S, H, 128, 128, generator=gen(seed), device=DEV) * 0.05).to(pool_dt)
    conv = torch.randn(S, C, 4, generator=gen(seed + 1), device=DEV)
    w = torch.randn(C, 4, generator=gen(seed + 2), device=DEV) * 0.3
    bias = torch.randn(C, generator=gen(seed + 3), device=DEV) * 0.1 if with_bias else None
    x = torch.randn(B, C, generator=gen(seed + 4), device=DEV).to(x_dt)
    a_raw, b_raw, A, dtb = raw_gates((B, H), H, torch.bfloat16, seed=seed + 5)
    slots = torch.randperm(S, generator=torch.Generator().manual_seed(seed))[:B]
    slots = slots.to(torch.int32).to(DEV)
    return pool, conv, w, bias, x, a_raw, b_raw, A, dtb, slots


def _separate(kern, pool, conv, slots, x, w, bias, a_raw, b_raw, A, dtb, H, G):
    B, C = x.shape
    co = torch.empty(B, C, device=DEV)
    kern.conv1d_decode(conv, slots, x, w, bias, co)
    q, k, v = torch.split(co, [G * 128, G * 128, H * 128], dim=-1)
    y = torch.empty(B, H, 128, device=DEV)
    kern.gdn_decode_raw(pool, slots, q.unflatten(-1, (G, 128)), k.unflatten(-1, (G, 128)),
                        v.unflatten(-1, (H, 128)), a_raw, b_raw, A, dtb, y)
    return y


def _bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


@pytest.mark.parametrize("pool_dt", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["f16-pool", "bf16-pool", "f32-pool"])
@pytest.mark.parametrize("x_dt", [torch.bfloat16, torch.float32], ids=["bf16-x", "f32-x"])
@pytest.mark.parametrize("H,G", [(8, 4), (8, 8)], ids=["hpg2", "hpg1"])
def test_fused_equals_conv_then_decode(kern, pool_dt, x_dt, H, G):
    B, S = 5, 9
    pool, conv, w, bias, x, a_raw, b_raw, A, dtb, slots = _setup(B, H, G, S, pool_dt, x_dt, 31)
    p1, c1, p2, c2 = pool.clone(), conv.clone(), pool.clone(), conv.clone()
    for step in range(3):
        xs = torch.roll(x, step, dims=1).contiguous()
        y_sep = _separate(kern, p1, c1, slots, xs, w, bias, a_raw, b_raw, A, dtb, H, G)
        y_fused = torch.empty(B, H, 128, device=DEV)
        kern.gdn_conv_decode_raw(p2, c2, slots, xs, w, bias, a_raw, b_raw, A, dtb, y_fused, G)
        assert torch.equal(_bits(y_fused), _bits(y_sep)), f"step {step}: y differs"
    assert torch.equal(_bits(p2), _bits(p1)), "states differ"
    assert torch.equal(_bits(c2), _bits(c1)), "conv windows differ"
    live = set(slots.tolist())
    idle = [s for s in range(S) if s not in live]
    assert torch.equal(_bits(p2[idle]), _bits(pool[idle]))
    assert torch.equal(_bits(c2[idle]), _bits(conv[idle]))


def test_fused_at_the_config_shape_without_bias(kern):
    B, H, G, S = 128, 32, 16, 160
    pool, conv, w, bias, x, a_raw, b_raw, A, dtb, slots = _setup(B, H, G, S, torch.float16,
                                                                 torch.bfloat16, 41,
                                                                 with_bias=False)
    p1, c1 = pool.clone(), conv.clone()
    y_sep = _separate(kern, p1, c1, slots, x, w, None, a_raw, b_raw, A, dtb, H, G)
    y_fused = torch.empty(B, H, 128, device=DEV)
    kern.gdn_conv_decode_raw(pool, conv, slots, x, w, None, a_raw, b_raw, A, dtb, y_fused, G)
    assert torch.equal(_bits(y_fused), _bits(y_sep))
    assert torch.equal(_bits(pool), _bits(p1)) and torch.equal(_bits(conv), _bits(c1))


def test_fused_rejects_what_it_cannot_run(kern):
    H, G, S = 8, 4, 6
    pool, conv, w, bias, x, a_raw, b_raw, A, dtb, slots = _setup(3, H, G, S, torch.float16,
                                                                 torch.bfloat16, 51)
    y = torch.empty(3, H, 128, device=DEV)
    dup = torch.tensor([1, 1, 2], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="distinct"):
        kern.gdn_conv_decode_raw(pool, conv, dup, x, w, bias, a_raw, b_raw, A, dtb, y, G)
    conv3 = torch.zeros(S, conv.size(1), 3, device=DEV)
    with pytest.raises(RuntimeError, match="conv_kernel == 4"):
        kern.gdn_conv_decode_raw(pool, conv3, slots, x, w[:, :3].contiguous(), bias, a_raw,
                                 b_raw, A, dtb, y, G)
    p4 = torch.zeros(S, 8, 128, 128, device=DEV, dtype=torch.float16)
    c4 = torch.zeros(S, 2 * 2 * 128 + 8 * 128, 4, device=DEV)
    x4 = torch.zeros(3, c4.size(1), device=DEV, dtype=torch.bfloat16)
    w4 = torch.zeros(c4.size(1), 4, device=DEV)
    with pytest.raises(RuntimeError, match="1 or 2 value heads"):
        kern.gdn_conv_decode_raw(p4, c4, slots, x4, w4, None, a_raw, b_raw, A, dtb, y, 2)
