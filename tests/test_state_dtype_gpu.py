"""fp16 / bf16 state pools against an fp32 pool, through the decode kernel.

Mirrors the reference's tests/test_state_dtype.py:100-177 at the kernel level
(the reference drives a whole GatedDeltaNet layer; here the same recurrence is
driven through gdn_decode_raw with seeded synthetic inputs): one step from the
same starting state moves the narrow pool's state only by storage rounding, and
over many free-running steps the rounding reaches a floor instead of
compounding.
"""
from __future__ import annotations

import pytest
import torch

from gpu_helpers import DEV, gen, raw_gates

pytestmark = pytest.mark.gpu
H, G, D = 32, 16, 128
NARROW = [torch.float16, torch.bfloat16]
IDS = ["fp16", "bf16"]


def _rel(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm()).item()


def _step_inputs(B, seed):
    g = gen(seed)
    q = torch.randn(B, G, D, generator=g, device=DEV)
    k = torch.randn(B, G, D, generator=g, device=DEV)
    v = torch.randn(B, H, D, generator=g, device=DEV)
    return q, k, v


@pytest.mark.parametrize("dt", NARROW, ids=IDS)
def test_one_step_from_the_same_state_moves_only_by_storage_rounding(kern, dt):
    """test_state_dtype.py:100-144: with the same starting state (as each pool
    represents it) one step differs from the fp32 pool by the storage type's
    rounding only; a scan narrowed to 16-bit arithmetic would miss this by
    orders of magnitude (the reductions run over 128 terms)."""
    B = 4
    seed_state = torch.randn(B, H, D, D, generator=gen(5), device=DEV) * 0.1
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    q, k, v = _step_inputs(B, 6)
    a, b, A, dtb = raw_gates((B, H), H, torch.bfloat16, seed=7)
    ys, states = {}, {}
    for name, sdt in (("fp32", torch.float32), ("narrow", dt)):
        pool = seed_state.to(sdt).clone()
        y = torch.empty(B, H, D, device=DEV)
        kern.gdn_decode_raw(pool, slots, q, k, v, a, b, A, dtb, y)
        ys[name], states[name] = y, pool.float()
    eps = torch.finfo(dt).eps
    rs = _rel(states["narrow"], states["fp32"])
    ry = _rel(ys["narrow"], ys["fp32"])
    # two roundings can land on one element: the seed cast and the store
    assert rs < 4 * eps, f"state moved {rs:.3e}, more than storage rounding ({eps:.1e})"
    assert ry < 40 * eps, f"output moved {ry:.3e}, more than storage rounding ({eps:.1e})"


@pytest.mark.parametrize("dt", NARROW, ids=IDS)
def test_drift_over_many_steps_stays_bounded(kern, dt):
    """test_state_dtype.py:147-177: alpha < 1 decays old state, so a per-step
    storage rounding must settle to a floor rather than ramp: the narrow pool's
    residual after 64 free-running steps is no worse than a small multiple of
    its residual after 8."""
    B, steps = 2, 64
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    start = torch.randn(B, H, D, D, generator=gen(9), device=DEV) * 0.05
    pools = {"fp32": start.clone(), "narrow": start.to(dt).contiguous()}
    _, _, A, dtb = raw_gates((B, H), H, torch.bfloat16, seed=10)
    at8 = None
    for t in range(steps):
        q, k, v = _step_inputs(B, 100 + t)
        a, b, _, _ = raw_gates((B, H), H, torch.bfloat16, seed=200 + t)
        for pool in pools.values():
            y = torch.empty(B, H, D, device=DEV)
            kern.gdn_decode_raw(pool, slots, q, k, v, a, b, A, dtb, y)
        if t == 7:
            at8 = _rel(pools["narrow"], pools["fp32"])
    at64 = _rel(pools["narrow"], pools["fp32"])
    assert at64 < max(4 * at8, 8 * torch.finfo(dt).eps), (
        f"drift grew from {at8:.3e} after 8 steps to {at64:.3e} after {steps}")
