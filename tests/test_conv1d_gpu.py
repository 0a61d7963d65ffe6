"""conv1d_decode on the GPU against the oracle (reference tests/test_conv1d_decode.py
and test_copy_kill.py:50-68)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import ATOL, DEV, RTOL, gen

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("K", [2, 3, 4, 8])
def test_matches_oracle_single_step(kern, K):
    C, B = 512, 3
    g = gen(1)
    p = torch.randn(8, C, K, generator=g, device=DEV)
    slots = torch.tensor([5, 0, 2], dtype=torch.int32, device=DEV)
    x = torch.randn(B, C, generator=g, device=DEV)
    w = torch.randn(C, K, generator=g, device=DEV)
    bias = torch.randn(C, generator=g, device=DEV)
    ref_pool = p.cpu().numpy().copy()
    out_ref = oracle.conv1d_decode(ref_pool, [5, 0, 2], x.cpu().numpy(), w.cpu().numpy(),
                                   bias.cpu().numpy())
    out = torch.empty(B, C, device=DEV)
    kern.conv1d_decode(p, slots, x, w, bias, out)
    np.testing.assert_allclose(out.cpu().numpy(), out_ref, rtol=RTOL, atol=ATOL)
    np.testing.assert_array_equal(p.cpu().numpy(), ref_pool)  # the window slide is exact


def test_matches_golden_fixture_without_and_with_bias(kern):
    gd = np.load(GOLDEN / "conv_f64.npz")
    p = torch.from_numpy(gd["window"]).to(DEV).contiguous()
    B, C = gd["x"].shape
    out = torch.empty(B, C, device=DEV)
    kern.conv1d_decode(p, torch.arange(B, dtype=torch.int32, device=DEV),
                       torch.from_numpy(gd["x"]).to(DEV), torch.from_numpy(gd["weight"]).to(DEV),
                       torch.from_numpy(gd["bias"]).to(DEV), out)
    np.testing.assert_allclose(out.cpu().numpy(), gd["out"], rtol=RTOL, atol=ATOL)
    np.testing.assert_array_equal(p.cpu().numpy(), gd["window_out"])
    # bias None and empty both mean "no bias"
    p2 = torch.from_numpy(gd["window"]).to(DEV).contiguous()
    p3 = p2.clone()
    o2, o3 = torch.empty(B, C, device=DEV), torch.empty(B, C, device=DEV)
    args = (torch.arange(B, dtype=torch.int32, device=DEV), torch.from_numpy(gd["x"]).to(DEV),
            torch.from_numpy(gd["weight"]).to(DEV))
    kern.conv1d_decode(p2, *args, None, o2)
    kern.conv1d_decode(p3, *args, torch.empty(0, device=DEV), o3)
    assert torch.equal(o2, o3)


def test_eight_steps_with_rotating_slots(kern):
    C, K, B, S = 256, 4, 4, 16
    g = gen(3)
    p = torch.randn(S, C, K, generator=g, device=DEV)
    ref_pool = p.cpu().numpy().copy()
    w = torch.randn(C, K, generator=g, device=DEV)
    bias = torch.randn(C, generator=g, device=DEV)
    out = torch.empty(B, C, device=DEV)
    for step in range(8):
        assignment = [(step * 3 + i) % S for i in range(B)]
        slots = torch.tensor(assignment, dtype=torch.int32, device=DEV)
        x = torch.randn(B, C, generator=g, device=DEV)
        out_ref = oracle.conv1d_decode(ref_pool, assignment, x.cpu().numpy(), w.cpu().numpy(),
                                       bias.cpu().numpy())
        kern.conv1d_decode(p, slots, x, w, bias, out)
        np.testing.assert_allclose(out.cpu().numpy(), out_ref, rtol=RTOL, atol=ATOL,
                                   err_msg=f"step {step}")
    np.testing.assert_array_equal(p.cpu().numpy(), ref_pool)


def test_silu_is_applied_to_every_channel(kern):
    C, K = 8192, 4
    p = torch.zeros(2, C, K, device=DEV)
    x = torch.full((1, C), -6.0, device=DEV)
    w = torch.zeros(C, K, device=DEV)
    w[:, -1] = 1.0
    out = torch.empty(1, C, device=DEV)
    kern.conv1d_decode(p, torch.tensor([0], dtype=torch.int32, device=DEV), x, w,
                       torch.zeros(C, device=DEV), out)
    expected = -6.0 / (1.0 + np.exp(6.0))
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=1e-6)


@pytest.mark.parametrize("B", [1, 6])
def test_bf16_input_equals_the_fp32_cast(kern, B):
    C, K = 8192, 4
    g = gen(3)
    x16 = torch.randn(B, C, generator=g, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(C, K, generator=g, device=DEV) * 0.3
    bias = torch.randn(C, generator=g, device=DEV) * 0.1
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    p1 = torch.randn(B, C, K, generator=g, device=DEV) * 0.2
    p2 = p1.clone()
    o1, o2 = torch.empty(B, C, device=DEV), torch.empty(B, C, device=DEV)
    kern.conv1d_decode(p1, slots, x16.float().contiguous(), w, bias, o1)
    kern.conv1d_decode(p2, slots, x16.contiguous(), w, bias, o2)
    assert torch.equal(o1, o2) and torch.equal(p1, p2)


def test_out_of_range_slot_is_rejected_duplicates_are_not(kern):
    C, K = 256, 4
    p = torch.zeros(4, C, K, device=DEV)
    x = torch.zeros(2, C, device=DEV)
    w = torch.zeros(C, K, device=DEV)
    out = torch.empty(2, C, device=DEV)
    with pytest.raises(RuntimeError, match="range"):
        kern.conv1d_decode(p, torch.tensor([0, 4], dtype=torch.int32, device=DEV), x, w, None, out)
    # the reference's conv checks range only (conv1d_decode.cu:77-89): a shared
    # scratch slot for padded graph rows is legal
    kern.conv1d_decode(p, torch.tensor([1, 1], dtype=torch.int32, device=DEV), x, w, None, out)


def test_graph_replay_survives_slot_reassignment(kern):
    C, K, B = 512, 4, 4
    p = torch.zeros(16, C, K, device=DEV)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    x = torch.zeros(B, C, device=DEV)
    g = gen(19)
    w = torch.randn(C, K, generator=g, device=DEV)
    bias = torch.randn(C, generator=g, device=DEV)
    out = torch.zeros(B, C, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            kern.conv1d_decode(p, slots, x, w, bias, out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kern.conv1d_decode(p, slots, x, w, bias, out)
    for assignment in ([9, 2, 15, 0], [1, 3, 5, 7]):
        p.normal_(generator=g)
        x.normal_(generator=g)
        slots.copy_(torch.tensor(assignment, dtype=torch.int32, device=DEV))
        ref_pool = p.cpu().numpy().copy()
        out_ref = oracle.conv1d_decode(ref_pool, assignment, x.cpu().numpy(), w.cpu().numpy(),
                                       bias.cpu().numpy())
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(out.cpu().numpy(), out_ref, rtol=RTOL, atol=ATOL)
        np.testing.assert_array_equal(p.cpu().numpy(), ref_pool)


# --- chunked prefill conv ----------------------------------------------------------

def _prefill_inputs(B, T, C, K, dt, seed):
    g = gen(seed)
    pool0 = torch.randn(B + 3, C, K, generator=g, device=DEV) * 0.5
    x = torch.randn(B, T, C, generator=g, device=DEV).to(dt)
    w = torch.randn(C, K, generator=g, device=DEV) * 0.3
    bias = torch.randn(C, generator=g, device=DEV) * 0.1
    return pool0, x, w, bias


@pytest.mark.parametrize("K", [2, 3, 4, 8])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32-x", "bf16-x"])
def test_prefill_equals_decode_token_by_token(kern, K, dt):
    B, T, C = 4, 21, 512
    pool0, x, w, bias = _prefill_inputs(B, T, C, K, dt, seed=K)
    slots = torch.tensor([5, 0, 3, 1], dtype=torch.int32, device=DEV)
    lens = torch.tensor([21, 0, 9, 40], dtype=torch.int32, device=DEV)  # full, empty, ragged, > T
    pp = pool0.clone()
    out = torch.full((B, T, C), float("nan"), device=DEV)
    kern.conv1d_prefill(pp, slots, x, w, bias, out, lens)
    pd = pool0.clone()
    lens_l = [min(max(int(n), 0), T) for n in lens.tolist()]
    for t in range(T):
        live = [b for b in range(B) if t < lens_l[b]]
        if not live:
            continue
        o = torch.empty(len(live), C, device=DEV)
        kern.conv1d_decode(pd, slots[live].contiguous(), x[live, t].contiguous(), w, bias, o)
        assert torch.equal(o, out[live, t]), f"token {t} differs from decode"
    assert torch.equal(pp, pd), "saved windows differ from decode applied per token"
    for b in range(B):
        assert (out[b, lens_l[b]:] == 0).all(), "pad positions must be written as 0"


def test_prefill_matches_oracle_and_saves_the_last_k_real_inputs(kern):
    B, T, C, K = 3, 17, 256, 4
    pool0, x, w, bias = _prefill_inputs(B, T, C, K, torch.bfloat16, seed=7)
    slots = torch.tensor([2, 4, 0], dtype=torch.int32, device=DEV)
    lens = torch.tensor([17, 5, 2], dtype=torch.int32, device=DEV)
    ref_pool = pool0.cpu().numpy().copy()
    out_ref = oracle.conv1d_prefill(ref_pool, slots.cpu().numpy(), x.float().cpu().numpy(),
                                    w.cpu().numpy(), bias.cpu().numpy(), lens.cpu().numpy())
    p = pool0.clone()
    out = torch.empty(B, T, C, device=DEV)
    kern.conv1d_prefill(p, slots, x, w, bias, out, lens)
    np.testing.assert_allclose(out.cpu().numpy(), out_ref, rtol=RTOL, atol=ATOL)
    np.testing.assert_array_equal(p.cpu().numpy(), ref_pool)
    # the saved window of a ragged row is its last K real inputs (here len 5)
    np.testing.assert_array_equal(p[4].cpu().numpy(), x[1, 1:5].float().t().cpu().numpy())


def test_prefill_rejects_duplicate_slots_and_handles_no_seq_lens(kern):
    B, T, C, K = 2, 5, 256, 4
    pool0, x, w, bias = _prefill_inputs(B, T, C, K, torch.float32, seed=9)
    out = torch.empty(B, T, C, device=DEV)
    with pytest.raises(RuntimeError, match="duplicate|distinct"):
        kern.conv1d_prefill(pool0.clone(), torch.tensor([1, 1], dtype=torch.int32, device=DEV),
                            x, w, bias, out)
    p1, p2 = pool0.clone(), pool0.clone()
    o1, o2 = torch.empty_like(out), torch.empty_like(out)
    slots = torch.tensor([1, 3], dtype=torch.int32, device=DEV)
    kern.conv1d_prefill(p1, slots, x, w, bias, o1, None)
    kern.conv1d_prefill(p2, slots, x, w, bias, o2,
                        torch.full((B,), T, dtype=torch.int32, device=DEV))
    assert torch.equal(o1, o2) and torch.equal(p1, p2)


def test_prefill_scalar_channel_path_equals_decode(kern):
    """C not a multiple of 4 takes the one-channel-per-thread path."""
    B, T, C, K = 2, 19, 258, 4
    pool0, x, w, bias = _prefill_inputs(B, T, C, K, torch.bfloat16, seed=21)
    slots = torch.tensor([3, 1], dtype=torch.int32, device=DEV)
    lens = torch.tensor([19, 7], dtype=torch.int32, device=DEV)
    pp, pd = pool0.clone(), pool0.clone()
    out = torch.empty(B, T, C, device=DEV)
    kern.conv1d_prefill(pp, slots, x, w, bias, out, lens)
    for t in range(T):
        live = [b for b in range(B) if t < int(lens[b])]
        o = torch.empty(len(live), C, device=DEV)
        kern.conv1d_decode(pd, slots[live].contiguous(), x[live, t].contiguous(), w, bias, o)
        assert torch.equal(o, out[live, t])
    assert torch.equal(pp, pd)
