"""gdn_decode / gdn_decode_raw on the GPU, through the C ABI, against the oracle.

Mirrors the reference's kernel gates (tests/test_gdn_decode_kernel.py,
test_slot_indirection.py, test_gdn_raw_gates.py:106-202, test_copy_kill.py:97-162)
with the CPU oracle as the checker instead of the reference's torch oracle.
"""
from __future__ import annotations

import time
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import (DEV, KIND, act_np, assert_parity, assert_pool_close, decode_inputs, gen,
                         pool, raw_gates, to_np_pool, torch_gates)

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
POOL_DTYPES = [torch.float32, torch.float16, torch.bfloat16]
POOL_IDS = ["f32-pool", "f16-pool", "bf16-pool"]


def _np(d):
    return {k: v.cpu().numpy() for k, v in d.items()}


@pytest.mark.parametrize("B", [1, 2, 8, 32])
def test_decode_matches_oracle(kern, B):
    p = pool(64)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    inp = decode_inputs(B)
    ref_pool = to_np_pool(p)
    n = _np(inp)
    y_ref = oracle.gdn_decode(ref_pool, np.arange(B), n["q"], n["k"], n["v"], n["alpha"],
                              n["beta"], "f32")
    y = torch.empty(B, 8, 128, device=DEV)
    kern.gdn_decode(p, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], y)
    assert_parity(y.cpu().numpy(), y_ref, 'y')
    assert_pool_close(p, ref_pool, slice(0, 64))


@pytest.mark.parametrize("dt", POOL_DTYPES, ids=POOL_IDS)
def test_decode_each_pool_dtype_matches_oracle(kern, dt):
    B = 8
    p = pool(20, dtype=dt, seed=5)
    slots = torch.tensor([19, 0, 7, 3, 12, 5, 11, 2], dtype=torch.int32, device=DEV)
    inp = decode_inputs(B, seed=6)
    ref_pool = to_np_pool(p)
    n = _np(inp)
    y_ref = oracle.gdn_decode(ref_pool, slots.cpu().numpy(), n["q"], n["k"], n["v"], n["alpha"],
                              n["beta"], KIND[dt])
    y = torch.empty(B, 8, 128, device=DEV)
    kern.gdn_decode(p, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], y)
    assert_parity(y.cpu().numpy(), y_ref, 'y')
    assert_pool_close(p, ref_pool, slice(0, 20), f"{dt} pool")


def test_decode_matches_golden_float64_fixture(kern):
    g = np.load(GOLDEN / "decode_f64.npz")
    p = torch.from_numpy(g["state"]).to(DEV).contiguous()
    t = {k: torch.from_numpy(g[k]).to(DEV).contiguous() for k in ("q", "k", "v", "alpha", "beta")}
    y = torch.empty(1, 2, 128, device=DEV)
    kern.gdn_decode(p, torch.zeros(1, dtype=torch.int32, device=DEV), t["q"], t["k"], t["v"],
                    t["alpha"], t["beta"], y)
    assert_parity(y.cpu().numpy(), g["y"], 'y')
    assert_parity(p.cpu().numpy(), g["state_out"], "fp32 state")


def test_nonidentity_slots_are_honoured_and_others_untouched(kern):
    p = pool(16, H=4)
    untouched = p.clone()
    slots = torch.tensor([7, 3], dtype=torch.int32, device=DEV)
    inp = decode_inputs(2, H=4, G=2)
    ref_pool = to_np_pool(p)
    n = _np(inp)
    y_ref = oracle.gdn_decode(ref_pool, [7, 3], n["q"], n["k"], n["v"], n["alpha"], n["beta"],
                              "f32")
    y = torch.empty(2, 4, 128, device=DEV)
    kern.gdn_decode(p, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], y)
    assert_parity(y.cpu().numpy(), y_ref, 'y')
    assert_pool_close(p, ref_pool, [7, 3])
    for s in (0, 1, 2, 4, 5, 6, 8, 15):
        assert torch.equal(p[s], untouched[s])


def test_rows_do_not_leak_into_each_other(kern):
    pa = pool(8)
    pb = pa.clone()
    two = decode_inputs(2, seed=11)
    y2 = torch.empty(2, 8, 128, device=DEV)
    kern.gdn_decode(pa, torch.tensor([0, 1], dtype=torch.int32, device=DEV), two["q"], two["k"],
                    two["v"], two["alpha"], two["beta"], y2)
    solo = {k: v[1:2].contiguous() for k, v in two.items()}
    y1 = torch.empty(1, 8, 128, device=DEV)
    kern.gdn_decode(pb, torch.tensor([1], dtype=torch.int32, device=DEV), solo["q"], solo["k"],
                    solo["v"], solo["alpha"], solo["beta"], y1)
    assert torch.equal(y2[1:2], y1)
    assert torch.equal(pa[1], pb[1])


def test_repeated_slot_is_rejected(kern):
    p = pool(8, H=4)
    inp = decode_inputs(2, H=4, G=2)
    y = torch.empty(2, 4, 128, device=DEV)
    with pytest.raises(RuntimeError, match="duplicate|distinct"):
        kern.gdn_decode(p, torch.tensor([2, 2], dtype=torch.int32, device=DEV), inp["q"],
                        inp["k"], inp["v"], inp["alpha"], inp["beta"], y)


def test_out_of_range_slot_is_rejected(kern):
    p = pool(8, H=4)
    inp = decode_inputs(2, H=4, G=2)
    y = torch.empty(2, 4, 128, device=DEV)
    for bad in ([0, 99], [-1, 0]):
        with pytest.raises(RuntimeError, match="range|bounds"):
            kern.gdn_decode(p, torch.tensor(bad, dtype=torch.int32, device=DEV), inp["q"],
                            inp["k"], inp["v"], inp["alpha"], inp["beta"], y)


def _strided_qkv(B, H=32, G=16, seed=7):
    """q/k/v as column slices of one [B, C] conv-output buffer (row stride C)."""
    C = 2 * G * 128 + H * 128
    buf = torch.randn(B, C, generator=gen(seed), device=DEV)
    q, k, v = torch.split(buf, [G * 128, G * 128, H * 128], dim=-1)
    return (q.unflatten(-1, (G, 128)), k.unflatten(-1, (G, 128)), v.unflatten(-1, (H, 128)))


@pytest.mark.parametrize("B", [1, 5])
def test_strided_qkv_equals_contiguous(kern, B):
    q, k, v = _strided_qkv(B)
    if B > 1:
        assert not q.is_contiguous()
    alpha = torch.rand(B, 32, generator=gen(9), device=DEV)
    beta = torch.rand(B, 32, generator=gen(10), device=DEV)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    p1, p2 = pool(B, H=32), pool(B, H=32)
    y1, y2 = torch.empty(B, 32, 128, device=DEV), torch.empty(B, 32, 128, device=DEV)
    kern.gdn_decode(p1, slots, q.contiguous(), k.contiguous(), v.contiguous(), alpha, beta, y1)
    kern.gdn_decode(p2, slots, q, k, v, alpha, beta, y2)
    assert torch.equal(y1, y2) and torch.equal(p1, p2)
    a_raw, b_raw, A, dtb = raw_gates((B, 32), 32, torch.bfloat16, seed=23)
    kern.gdn_decode_raw(p1, slots, q.contiguous(), k.contiguous(), v.contiguous(), a_raw, b_raw,
                        A, dtb, y1)
    kern.gdn_decode_raw(p2, slots, q, k, v, a_raw, b_raw, A, dtb, y2)
    assert torch.equal(y1, y2) and torch.equal(p1, p2)


@pytest.mark.parametrize("pool_dt", POOL_DTYPES, ids=POOL_IDS)
@pytest.mark.parametrize("act", [torch.float32, torch.bfloat16], ids=["f32-act", "bf16-act"])
@pytest.mark.parametrize("B", [1, 5])
def test_raw_gates_equal_the_torch_computed_ones_bitwise(kern, B, act, pool_dt):
    inp = decode_inputs(B, H=32, G=16, seed=3)
    a_raw, b_raw, A, dtb = raw_gates((B, 32), 32, act)
    alpha, beta = torch_gates(a_raw, b_raw, A, dtb)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    p1, p2 = pool(B, H=32, dtype=pool_dt), pool(B, H=32, dtype=pool_dt)
    y1, y2 = torch.empty(B, 32, 128, device=DEV), torch.empty(B, 32, 128, device=DEV)
    kern.gdn_decode(p1, slots, inp["q"], inp["k"], inp["v"], alpha, beta, y1)
    kern.gdn_decode_raw(p2, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dtb, y2)
    assert torch.equal(y1, y2), f"outputs differ by {(y1 - y2).abs().max().item():.3e}"
    assert torch.equal(p1, p2), "states differ"


def test_raw_gates_match_the_oracle_gates(kern):
    """The in-kernel gates against the oracle's gate restatement, and the raw
    decode against the oracle at the parity bar. The oracle's recurrence is
    fed torch-ROCm's gates (gdn.py:299-300), which the in-kernel gates equal
    bit for bit (test_raw_gates_equal_the_torch_computed_ones_bitwise), so y
    and the fp32 state are held to max-abs 2e-5. The oracle's own gates, a
    host transcendental implementation, agree with them to the bars that pin
    the oracle against torch's CPU spelling (log alpha to 4e-7 relative; the
    bf16-rounded beta equal or one bf16 ulp apart)."""
    B, H = 4, 32
    inp = decode_inputs(B, H=H, G=16, seed=13)
    a_raw, b_raw, A, dtb = raw_gates((B, H), H, torch.bfloat16, seed=14)
    ref_pool = to_np_pool(pool(B, H=H))
    p = pool(B, H=H)
    al, be = oracle.gdn_gates(act_np(a_raw), act_np(b_raw), A.cpu().numpy(),
                              dtb.cpu().numpy(), "bf16")
    ta, tb = torch_gates(a_raw, b_raw, A, dtb)
    np.testing.assert_allclose(np.log(ta.cpu().numpy()), np.log(al), rtol=4e-7, atol=2e-7)
    assert (np.abs(tb.cpu().numpy() - be) <= np.abs(be) * 2 ** -7).all()
    n = _np(inp)
    y_ref = oracle.gdn_decode(ref_pool, np.arange(B), n["q"], n["k"], n["v"],
                              ta.cpu().numpy(), tb.cpu().numpy(), "f32")
    y = torch.empty(B, H, 128, device=DEV)
    kern.gdn_decode_raw(p, torch.arange(B, dtype=torch.int32, device=DEV), inp["q"], inp["k"],
                        inp["v"], a_raw, b_raw, A, dtb, y)
    assert_parity(y.cpu().numpy(), y_ref, "y (raw gates)")
    assert_parity(p.cpu().numpy(), ref_pool, "fp32 state (raw gates)")


def test_softplus_threshold_branch_matches_torch(kern):
    B, H = 1, 32
    inp = decode_inputs(B, H=H, G=16, seed=21)
    _, b_raw, A, _ = raw_gates((B, H), H, torch.float32, seed=23)
    dtb = torch.zeros(H, device=DEV)
    a_raw = torch.zeros(B, H, device=DEV)
    probes = [-80.0, -20.0, 0.0, 19.0, 19.999999, 20.0, 20.000001, 25.0, 80.0]
    a_raw[0, : len(probes)] = torch.tensor(probes, device=DEV)
    alpha, beta = torch_gates(a_raw, b_raw, A, dtb)
    slots = torch.zeros(1, dtype=torch.int32, device=DEV)
    p1, p2 = pool(1, H=H), pool(1, H=H)
    y1, y2 = torch.empty(1, H, 128, device=DEV), torch.empty(1, H, 128, device=DEV)
    kern.gdn_decode(p1, slots, inp["q"], inp["k"], inp["v"], alpha, beta, y1)
    kern.gdn_decode_raw(p2, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dtb, y2)
    assert torch.equal(y1, y2) and torch.equal(p1, p2), "gates differ across the threshold"


def _capture(kern, fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def test_graph_replay_survives_slot_reassignment(kern):
    B, H = 4, 8
    p = torch.zeros(32, H, 128, 128, device=DEV)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    q = torch.zeros(B, 4, 128, device=DEV)
    k = torch.zeros(B, 4, 128, device=DEV)
    v = torch.zeros(B, H, 128, device=DEV)
    alpha = torch.zeros(B, H, device=DEV)
    beta = torch.zeros(B, H, device=DEV)
    y = torch.zeros(B, H, 128, device=DEV)
    graph = _capture(kern, lambda: kern.gdn_decode(p, slots, q, k, v, alpha, beta, y))
    g = gen(7)
    for assignment in ([5, 9, 1, 30], [0, 1, 2, 3], [31, 2, 17, 8]):
        p.normal_(generator=g)
        q.normal_(generator=g)
        k.normal_(generator=g)
        v.normal_(generator=g)
        alpha.uniform_(0.5, 1.0, generator=g)
        beta.uniform_(0.0, 1.0, generator=g)
        slots.copy_(torch.tensor(assignment, dtype=torch.int32, device=DEV))
        ref_pool = to_np_pool(p)
        y_ref = oracle.gdn_decode(ref_pool, assignment, q.cpu().numpy(), k.cpu().numpy(),
                                  v.cpu().numpy(), alpha.cpu().numpy(), beta.cpu().numpy(), "f32")
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(y.cpu().numpy(), y_ref, 'y')
        assert_pool_close(p, ref_pool, slice(0, 32))


def test_replay_with_rotating_slots_is_cheap(kern):
    B, H = 8, 32
    p = pool(32, H=H)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    inp = decode_inputs(B, H=H, G=16)
    y = torch.empty(B, H, 128, device=DEV)
    graph = _capture(kern, lambda: kern.gdn_decode(p, slots, inp["q"], inp["k"], inp["v"],
                                                   inp["alpha"], inp["beta"], y))
    rotations = [torch.tensor([(i + r) % 32 for i in range(B)], dtype=torch.int32, device=DEV)
                 for r in range(8)]
    torch.cuda.synchronize()
    t = time.perf_counter()
    for r in range(200):
        slots.copy_(rotations[r % 8])
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t) / 200 * 1e3
    print(f"\n  rotating replay {ms:.4f} ms/step")
    assert ms < 1.0


@pytest.mark.parametrize("dt", POOL_DTYPES, ids=POOL_IDS)
def test_state_narrowing_rounds_to_nearest_even_exactly(kern, dt):
    """With beta = 0 the new state is exactly fl32(alpha * S) (the update adds a
    signed zero), narrowed once to the pool type. That value is fixed by IEEE
    arithmetic, so the pool must match it BITWISE: a truncating or otherwise
    mis-rounding narrowing fails here, where the 1-ulp oracle bars could not
    see it."""
    B, H = 4, 8
    p = pool(B, H=H, dtype=dt, seed=17, scale=1.0)
    before = p.float().cpu().numpy()
    inp = decode_inputs(B, H=H, seed=18)
    inp["beta"].zero_()
    y = torch.empty(B, H, 128, device=DEV)
    kern.gdn_decode(p, torch.arange(B, dtype=torch.int32, device=DEV), inp["q"], inp["k"],
                    inp["v"], inp["alpha"], inp["beta"], y)
    prod = (before * inp["alpha"].cpu().numpy()[:, :, None, None]).astype(np.float32)
    expected = oracle.narrow(prod, KIND[dt])
    got = to_np_pool(p)
    if dt == torch.float32:
        assert np.array_equal(got, expected)
    else:
        assert np.array_equal(got.view(np.uint16), expected.view(np.uint16)), (
            f"{int((got.view(np.uint16) != expected.view(np.uint16)).sum())} elements "
            "rounded differently from round-to-nearest-even")


@pytest.mark.parametrize("H,G", [(32, 16), (12, 4)], ids=["H32", "H12-tiles-not-mult-8"])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["f16-pool", "bf16-pool", "f32-pool"])
def test_launch_shapes_give_identical_bits(kern, dt, H, G):
    """A large launch (at least 8 tiles per CU on a 16-bit pool, 12 on fp32)
    walks XCD-contiguous tile ranges and, on a 16-bit pool, keeps two
    workgroups resident per CU (with the two-waves-per-SIMD build). Each tile is
    still one workgroup's work, so every launch shape (forced through the
    override variables) must leave the same pool and y bits; the default one is
    also checked against the oracle on a sample of rows. With H = 12 the tile
    count is not a multiple of 8, so the default large launch keeps dispatch
    order (and the cap)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    B = max(128, -(-12 * cus // H))
    B += (-B) % 8 if H % 8 == 0 else (1 - (B * H // 4) % 2)
    slots = torch.randperm(B + 16, generator=torch.Generator().manual_seed(3))[:B]
    slots = slots.to(torch.int32).to(DEV)
    inp = decode_inputs(B, H=H, G=G, seed=21)
    a_raw, b_raw, A, dt_bias = raw_gates((B, H), H, torch.bfloat16, seed=22)
    base = pool(B + 16, H=H, dtype=dt, seed=23)
    results = {}
    for label, remap, cap in (("default", None, None), ("dispatch order", 0, 0),
                              ("remap only", 1, 0), ("cap 2", 1, 2),
                              ("cap 4, dispatch order", 0, 4)):
        p = base.clone()
        y = torch.empty(B, H, 128, device=DEV)
        with kern.launch_override(decode_xcd_remap=remap, decode_wgs_per_cu=cap):
            kern.gdn_decode_raw(p, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dt_bias,
                                y)
        torch.cuda.synchronize()
        results[label] = (p, y)
    p0, y0 = results["default"]
    for label, (p, y) in results.items():
        assert torch.equal(p.view(torch.uint8), p0.view(torch.uint8)), label
        assert torch.equal(y, y0), label
    rows = [0, B // 2, B - 1]
    sub = slots[rows].cpu().numpy()
    if H % 8:
        assert (B * H) % 8 != 0
    ref_pool = to_np_pool(base)
    alpha, beta = torch_gates(a_raw, b_raw, A, dt_bias)
    n = {k: v[rows].cpu().numpy() for k, v in inp.items()}
    y_ref = oracle.gdn_decode(ref_pool, sub, n["q"], n["k"], n["v"],
                              alpha[rows].cpu().numpy(), beta[rows].cpu().numpy(), KIND[dt])
    assert_parity(y0[rows].cpu().numpy(), y_ref, 'y')


@pytest.mark.parametrize("dt", POOL_DTYPES, ids=POOL_IDS)
@pytest.mark.parametrize("B", [1, 3, 8])
def test_column_parts_give_identical_bits(kern, dt, B):
    """Small launches split each tile's columns over 2 or 4 workgroups (the
    decode_parts knob forces 1, 2 or 4). A column's rows, chains and
    reduction tree do not change, so every split must leave the same pool
    and y bits as one workgroup per tile; the default launch is also checked
    against the oracle (torch's gate spelling, max-abs 2e-5)."""
    H, G = 32, 16
    slots = torch.randperm(B + 5, generator=torch.Generator().manual_seed(B))[:B]
    slots = slots.to(torch.int32).to(DEV)
    inp = decode_inputs(B, H=H, G=G, seed=40 + B)
    a_raw, b_raw, A, dt_bias = raw_gates((B, H), H, torch.bfloat16, seed=41)
    base = pool(B + 5, H=H, dtype=dt, seed=42)
    results = {}
    for parts in (None, 1, 2, 4):
        p = base.clone()
        y = torch.empty(B, H, 128, device=DEV)
        with kern.launch_override(decode_parts=parts):
            kern.gdn_decode_raw(p, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dt_bias,
                                y)
        torch.cuda.synchronize()
        results[parts] = (p, y)
    p0, y0 = results[1]
    for parts, (p, y) in results.items():
        assert torch.equal(p.view(torch.uint8), p0.view(torch.uint8)), parts
        assert torch.equal(y, y0), parts
    pd, yd = results[None]
    alpha, beta = torch_gates(a_raw, b_raw, A, dt_bias)
    ref_pool = to_np_pool(base)
    n = {k: v.cpu().numpy() for k, v in inp.items()}
    y_ref = oracle.gdn_decode(ref_pool, slots.cpu().numpy(), n["q"], n["k"], n["v"],
                              alpha.cpu().numpy(), beta.cpu().numpy(), KIND[dt])
    assert_parity(yd.cpu().numpy(), y_ref, f"y, B={B}, default parts")
    assert_pool_close(pd, ref_pool, slice(0, B + 5), f"{dt} pool, B={B}")
