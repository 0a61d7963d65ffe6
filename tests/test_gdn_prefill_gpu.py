"""gdn_prefill / gdn_prefill_raw on the GPU, through the C ABI.

Mirrors the reference's chunk-scan gates (tests/test_gdn_prefill_kernel.py:84-206,
test_gdn_raw_gates.py:150-256): the chunk equals the decode kernel applied T
times bit for bit — here for fp32, fp16 AND bf16 pools, because the chunk
keeps its on-chip state in the pool's storage type — a pad column is an exact
identity, chunking is invisible, and raw gates / seq_lens equal the torch
spelling bit for bit. Plus parity with the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import (DEV, KIND, assert_free_running_close, assert_parity, assert_pool_close,
                         pool, prefill_inputs, raw_gates, to_np_pool, torch_gates)

pytestmark = pytest.mark.gpu
POOL_DTYPES = [torch.float32, torch.float16, torch.bfloat16]
POOL_IDS = ["f32-pool", "f16-pool", "bf16-pool"]


def _decode_t_times(kern, p, slots, q, k, v, alpha, beta):
    B, T = q.shape[:2]
    H = v.size(2)
    y = torch.empty(B, T, H, 128, device=DEV)
    for t in range(T):
        out = torch.empty(B, H, 128, device=DEV)
        kern.gdn_decode(p, slots, q[:, t].contiguous(), k[:, t].contiguous(),
                        v[:, t].contiguous(), alpha[:, t].contiguous(), beta[:, t].contiguous(),
                        out)
        y[:, t] = out
    return y


@pytest.mark.parametrize("T", [1, 4, 17, 128])
@pytest.mark.parametrize("B", [1, 5])
def test_chunk_equals_decode_applied_t_times(kern, T, B):
    inp = prefill_inputs(B, T, H=32, G=16)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    pc = pool(B, H=32)
    yc = torch.empty(B, T, 32, 128, device=DEV)
    kern.gdn_prefill(pc, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], yc)
    ps = pool(B, H=32)
    ys = _decode_t_times(kern, ps, slots, **inp)
    assert torch.equal(yc, ys), f"outputs differ by {(yc - ys).abs().max().item():.3e}"
    assert torch.equal(pc, ps), f"states differ by {(pc - ps).abs().max().item():.3e}"


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16], ids=["f16-pool", "bf16-pool"])
def test_a_narrow_pool_chunk_is_bit_identical_to_decode(kern, dt):
    """Stronger than the reference (which allowed 8 eps here): the chunk rounds
    its on-chip state through the pool type after every token, as T decode
    launches do, so the two are the same computation."""
    B, T = 3, 24
    inp = prefill_inputs(B, T, seed=9)
    slots = torch.tensor([4, 0, 2], dtype=torch.int32, device=DEV)
    pc = pool(6, dtype=dt)
    yc = torch.empty(B, T, 8, 128, device=DEV)
    kern.gdn_prefill(pc, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], yc)
    ps = pool(6, dtype=dt)
    ys = _decode_t_times(kern, ps, slots, **inp)
    assert torch.equal(yc, ys) and torch.equal(pc, ps)


@pytest.mark.parametrize("dt", POOL_DTYPES, ids=POOL_IDS)
def test_chunk_matches_oracle(kern, dt):
    B, T = 3, 17
    inp = prefill_inputs(B, T, seed=12)
    slots = torch.tensor([5, 1, 3], dtype=torch.int32, device=DEV)
    p = pool(6, dtype=dt, seed=13)
    ref_pool = to_np_pool(p)
    n = {k: v.cpu().numpy() for k, v in inp.items()}
    y_ref = oracle.gdn_prefill(ref_pool, [5, 1, 3], n["q"], n["k"], n["v"], n["alpha"],
                               n["beta"], KIND[dt])
    y = torch.empty(B, T, 8, 128, device=DEV)
    kern.gdn_prefill(p, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], y)
    # errors stay at one rounding per token: the update is non-expansive
    # (alpha <= 1, I - beta k k^T with |k| = 1 and beta in [0, 1])
    # fp32 pools: the stated max-abs bar. Narrow pools store the state after
    # every token, where a rounding tie may fall one ulp apart on the two
    # sides and is then carried forward: y is held to 1e-3 max-abs and to the
    # relative bar rtol 1e-4 / atol 1e-5 over the 17 tokens.
    if dt == torch.float32:
        assert_parity(y.cpu().numpy(), y_ref, "y (f32 pool, 17 tokens)", rel=False)
    else:
        assert_parity(y.cpu().numpy(), y_ref, f"y ({KIND[dt]} pool, 17 tokens)", maxabs=1e-3,
                      rel=False)
        np.testing.assert_allclose(y.cpu().numpy(), y_ref, rtol=1e-4, atol=1e-5)
    if dt == torch.float32:
        assert_parity(p.cpu().numpy(), ref_pool, "fp32 state (17 tokens)", rel=False)
    else:
        assert_free_running_close(to_np_pool(p), ref_pool, KIND[dt])


@pytest.mark.parametrize("dt", [torch.float32, torch.float16], ids=["f32-pool", "f16-pool"])
def test_a_long_chunk_matches_oracle_on_sampled_heads(kern, dt):
    """640 tokens with raw gates and ragged lengths, checked against the oracle
    on sampled (row, head) tiles. fp32 pool: y and the final state to max-abs
    2e-5. fp16 pool: the state within the free-running bound, and y to 1e-3:
    the two sides store the state through fp16 after every token, a rounding
    tie may fall one ulp apart (the per-step bar), and such a difference is
    carried forward, not amplified, by the non-expansive update. The oracle
    runs the sampled heads alone (H = G = 1), fed torch's gate spelling, which
    the in-kernel gates equal bit for bit."""
    B, T, H, Gk = 2, 640, 32, 16
    inp = prefill_inputs(B, T, H=H, G=Gk, seed=61)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=62)
    lens = torch.tensor([T, 517], dtype=torch.int32, device=DEV)
    slots = torch.tensor([2, 0], dtype=torch.int32, device=DEV)
    p = pool(3, H=H, dtype=dt, seed=63)
    before = to_np_pool(p)
    y = torch.empty(B, T, H, 128, device=DEV)
    kern.gdn_prefill_raw(p, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, y, lens)
    torch.cuda.synchronize()
    alpha, beta = torch_gates(a, b, A, dtb)
    after = to_np_pool(p)
    for row, head in ((0, 0), (0, 21), (1, 31)):
        n = int(lens[row])
        grp = head // (H // Gk)
        sub = before[int(slots[row]), head][None, None].copy()
        sl = lambda t, idx: t[row:row + 1, :n, idx:idx + 1].cpu().numpy()
        y_ref = oracle.gdn_prefill(sub, [0], sl(inp["q"], grp), sl(inp["k"], grp),
                                   sl(inp["v"], head), sl(alpha, head), sl(beta, head), KIND[dt])
        assert_parity(y[row:row + 1, :n, head:head + 1].cpu().numpy(), y_ref,
                      f"y row {row} head {head}, {n} tokens ({KIND[dt]} pool)",
                      maxabs=2e-5 if dt == torch.float32 else 1e-3, rel=False)
        got = after[int(slots[row]), head]
        if dt == torch.float32:
            assert_parity(got, sub[0, 0], f"fp32 state row {row} head {head}", rel=False)
        else:
            assert_free_running_close(got, sub[0, 0], KIND[dt])
    assert bool((y[1, 517:] == 0).all()), "pad outputs are not 0"


def test_a_pad_column_does_not_move_the_state(kern):
    B, T = 4, 6
    inp = prefill_inputs(B, T, seed=21)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    lens = torch.tensor([2, 3, 4, 6], device=DEV)
    live = (torch.arange(T, device=DEV)[None] < lens[:, None])[:, :, None]
    am = torch.where(live, inp["alpha"], 1.0).contiguous()
    bm = torch.where(live, inp["beta"], 0.0).contiguous()
    padded = pool(B)
    y = torch.empty(B, T, 8, 128, device=DEV)
    kern.gdn_prefill(padded, slots, inp["q"], inp["k"], inp["v"], am, bm, y)
    for b in range(B):
        n = int(lens[b])
        solo = pool(B)[b:b + 1].contiguous()
        y1 = torch.empty(1, n, 8, 128, device=DEV)
        kern.gdn_prefill(solo, torch.zeros(1, dtype=torch.int32, device=DEV),
                         inp["q"][b:b + 1, :n].contiguous(), inp["k"][b:b + 1, :n].contiguous(),
                         inp["v"][b:b + 1, :n].contiguous(), am[b:b + 1, :n].contiguous(),
                         bm[b:b + 1, :n].contiguous(), y1)
        assert torch.equal(padded[b], solo[0]), f"row {b} state moved under padding"
        assert torch.equal(y[b, :n], y1[0]), f"row {b} outputs moved"


@pytest.mark.parametrize("cut", [1, 7, 64])
def test_two_chunks_leave_the_same_state_as_one(kern, cut):
    B, T = 2, 96
    inp = prefill_inputs(B, T, seed=33)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    whole = pool(B)
    yw = torch.empty(B, T, 8, 128, device=DEV)
    kern.gdn_prefill(whole, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], yw)
    parts = pool(B)
    yp = torch.empty(B, T, 8, 128, device=DEV)
    for lo, hi in ((0, cut), (cut, T)):
        out = torch.empty(B, hi - lo, 8, 128, device=DEV)
        kern.gdn_prefill(parts, slots, *(inp[n][:, lo:hi].contiguous()
                                         for n in ("q", "k", "v", "alpha", "beta")), out)
        yp[:, lo:hi] = out
    assert torch.equal(whole, parts) and torch.equal(yw, yp)


@pytest.mark.parametrize("act", [torch.float32, torch.bfloat16], ids=["f32-act", "bf16-act"])
@pytest.mark.parametrize("T", [1, 17, 96])
def test_prefill_raw_gates_equal_the_torch_computed_ones(kern, T, act):
    B = 3
    inp = prefill_inputs(B, T, H=32, G=16, seed=31)
    a_raw, b_raw, A, dtb = raw_gates((B, T, 32), 32, act, seed=33)
    alpha, beta = torch_gates(a_raw, b_raw, A, dtb)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    p1, p2 = pool(B, H=32), pool(B, H=32)
    y1, y2 = torch.empty(B, T, 32, 128, device=DEV), torch.empty(B, T, 32, 128, device=DEV)
    kern.gdn_prefill(p1, slots, inp["q"], inp["k"], inp["v"], alpha, beta, y1)
    kern.gdn_prefill_raw(p2, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dtb, y2, None)
    assert torch.equal(y1, y2) and torch.equal(p1, p2)


def test_seq_lens_is_the_where_mask_bit_for_bit(kern):
    """seq_lens gives the states and the live outputs of the reference's
    where-mask (gdn.py:313-316) bit for bit. The kernel skips the pad steps
    (exact identities) and writes 0 at the pad outputs, which the reference
    leaves unspecified."""
    B, T = 4, 12
    inp = prefill_inputs(B, T, H=32, G=16, seed=41)
    a_raw, b_raw, A, dtb = raw_gates((B, T, 32), 32, torch.bfloat16, seed=43)
    alpha, beta = torch_gates(a_raw, b_raw, A, dtb)
    lens = torch.tensor([3, 7, 12, 1], device=DEV, dtype=torch.int32)
    live = (torch.arange(T, device=DEV)[None] < lens[:, None])[:, :, None]
    am = torch.where(live, alpha, 1.0).contiguous()
    bm = torch.where(live, beta, 0.0).contiguous()
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    p1, p2 = pool(B, H=32), pool(B, H=32)
    y1, y2 = torch.empty(B, T, 32, 128, device=DEV), torch.empty(B, T, 32, 128, device=DEV)
    kern.gdn_prefill(p1, slots, inp["q"], inp["k"], inp["v"], am, bm, y1)
    kern.gdn_prefill_raw(p2, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dtb, y2, lens)
    assert torch.equal(p1, p2)
    lv = live[:, :, 0]
    assert torch.equal(y1[lv], y2[lv])
    assert bool((y2[~lv] == 0).all()), "pad outputs must be 0"


def test_a_len_of_zero_and_a_len_beyond_t_are_legal(kern):
    B, T = 2, 6
    inp = prefill_inputs(B, T, H=32, G=16, seed=51)
    a_raw, b_raw, A, dtb = raw_gates((B, T, 32), 32, torch.float32, seed=53)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    lens = torch.tensor([0, T + 5], device=DEV, dtype=torch.int32)
    p = pool(B, H=32)
    before = p[0].clone()
    y = torch.empty(B, T, 32, 128, device=DEV)
    kern.gdn_prefill_raw(p, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dtb, y, lens)
    assert torch.equal(p[0], before)
    assert bool((y[0] == 0).all()), "a row of length 0 outputs zeros"
    pr = pool(B, H=32)
    yr = torch.empty_like(y)
    kern.gdn_prefill_raw(pr, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dtb, yr, None)
    assert torch.equal(p[1], pr[1]) and torch.equal(y[1], yr[1])


def test_prefill_rejects_duplicate_slots(kern):
    inp = prefill_inputs(2, 3)
    p = pool(4)
    y = torch.empty(2, 3, 8, 128, device=DEV)
    with pytest.raises(RuntimeError, match="duplicate|distinct"):
        kern.gdn_prefill(p, torch.tensor([1, 1], dtype=torch.int32, device=DEV), inp["q"],
                         inp["k"], inp["v"], inp["alpha"], inp["beta"], y)


def _same_up_to_zero_sign(a, b, dt):
    """Bitwise equal, except that -0 on one side may be +0 on the other."""
    ib = (lambda t: t.view(torch.int32)) if dt == torch.float32 else (lambda t: t.view(torch.int16))
    diff = ib(a) != ib(b)
    return bool((~diff | ((a == 0) & (b == 0))).all())


@pytest.mark.parametrize("dt", POOL_DTYPES, ids=POOL_IDS)
def test_identity_steps_are_exact_up_to_the_sign_of_zero(kern, dt):
    """alpha = 1, beta = 0 (a pad step) leaves every state element's bits alone
    except that 1*(-0) + 0 = +0: the reference's own arithmetic
    (gdn_decode.cu:120-124, S' = a*S + k*delta), whose tests compare with
    torch.equal, where -0 == +0. Checked with negative zeros planted in the
    pool, for a caller-padded chunk, a single decode step and a ragged raw-gates
    chunk against decode over the live tokens only."""
    B, T = 2, 6
    p0 = pool(4, dtype=dt, seed=21)
    p0.view(-1)[::7] = -0.0
    slots = torch.tensor([3, 1], dtype=torch.int32, device=DEV)

    inp = prefill_inputs(B, T, seed=22)
    inp["alpha"].fill_(1.0)
    inp["beta"].zero_()
    p = p0.clone()
    y = torch.empty(B, T, 8, 128, device=DEV)
    kern.gdn_prefill(p, slots, inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], y)
    assert torch.equal(p, p0) and _same_up_to_zero_sign(p, p0, dt)

    p = p0.clone()
    out = torch.empty(B, 8, 128, device=DEV)
    kern.gdn_decode(p, slots, inp["q"][:, 0].contiguous(), inp["k"][:, 0].contiguous(),
                    inp["v"][:, 0].contiguous(), inp["alpha"][:, 0].contiguous(),
                    inp["beta"][:, 0].contiguous(), out)
    assert torch.equal(p, p0) and _same_up_to_zero_sign(p, p0, dt)

    a_raw, b_raw, A, dt_bias = raw_gates((B, T, 8), 8, torch.bfloat16, seed=23)
    lens = torch.tensor([2, 0], dtype=torch.int32, device=DEV)
    pr = p0.clone()
    kern.gdn_prefill_raw(pr, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dt_bias, y,
                         lens)
    pd = p0.clone()
    for t in range(2):
        o = torch.empty(1, 8, 128, device=DEV)
        kern.gdn_decode_raw(pd, slots[:1], inp["q"][:1, t].contiguous(),
                            inp["k"][:1, t].contiguous(), inp["v"][:1, t].contiguous(),
                            a_raw[:1, t].contiguous(), b_raw[:1, t].contiguous(), A, dt_bias, o)
    assert torch.equal(pr, pd) and _same_up_to_zero_sign(pr, pd, dt)


@pytest.mark.parametrize("cols", [1, 2, 0, 4, 8],
                         ids=["split-1col", "whole-2col", "planned", "quarter", "eighth"])
@pytest.mark.parametrize("dt", POOL_DTYPES, ids=POOL_IDS)
def test_both_scan_layouts_are_decode_bit_for_bit(kern, dt, cols):
    """The launch picks one column per lane (a tile split over two workgroups)
    for small launches, two otherwise, or, for larger ragged batches, a plan
    per row; the quarter and eighth layouts (one column and 16 or 8 rows per
    lane, a tile over four or eight workgroups) serve the smallest launches
    (the prefill_layout knob = 1, 2, 0, 4 or 8 forces each; here the planned
    launch splits the 40-token row and runs the others whole). Every layout
    must equal decode applied T times, with raw gates and ragged seq_lens
    including 0, on every pool type, with zeros at the pad outputs."""
    B, T, H, G = 3, 40, 32, 16
    inp = prefill_inputs(B, T, H=H, G=G, seed=21)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=22)
    lens = torch.tensor([40, 0, 23], dtype=torch.int32, device=DEV)
    slots = torch.tensor([5, 1, 3], dtype=torch.int32, device=DEV)
    pc = pool(7, H=H, dtype=dt)
    ps = pc.clone()
    yc = torch.empty(B, T, H, 128, device=DEV)
    with kern.launch_override(prefill_layout=cols):
        kern.gdn_prefill_raw(pc, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yc, lens)
    for t in range(T):
        live = (t < lens).nonzero().flatten()
        if live.numel() == 0:
            continue
        yt = torch.empty(live.numel(), H, 128, device=DEV)
        kern.gdn_decode_raw(ps, slots[live].contiguous(), inp["q"][live, t].contiguous(),
                            inp["k"][live, t].contiguous(), inp["v"][live, t].contiguous(),
                            a[live, t].contiguous(), b[live, t].contiguous(), A, dtb, yt)
        assert torch.equal(yc[live, t], yt), f"token {t}: outputs differ"
        dead = (t >= lens).nonzero().flatten()
        assert bool((yc[dead, t] == 0).all()), f"token {t}: pad outputs are not 0"
    assert bool((yc[1] == 0).all())
    torch.cuda.synchronize()
    same = (pc == ps) | (pc.isnan() & ps.isnan())
    assert bool(same.all()), f"states differ by {(pc.float() - ps.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("cols", [1, 2, 0, 4, 8],
                         ids=["split-1col", "whole-2col", "planned", "quarter", "eighth"])
def test_stage_boundaries_are_decode_bit_for_bit(kern, cols):
    """Row lengths around the 32-token stage and the token-pair loops' tails:
    33 (a second stage of one token), 64 (two full stages), 34 and 35 (a
    second stage of a pair, and of a pair and one), 1 and 31 (one stage, a
    single token / an odd tail). Each layout must equal decode applied token
    by token, bit for bit, with zeros at the pad outputs."""
    lens_l = [33, 64, 34, 1, 35, 31]
    B, T, H, G = len(lens_l), max(lens_l), 32, 16
    inp = prefill_inputs(B, T, H=H, G=G, seed=91)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=92)
    lens = torch.tensor(lens_l, dtype=torch.int32, device=DEV)
    slots = torch.tensor([7, 2, 0, 5, 3, 8], dtype=torch.int32, device=DEV)
    pc = pool(10, H=H, dtype=torch.float16)
    ps = pc.clone()
    yc = torch.empty(B, T, H, 128, device=DEV)
    with kern.launch_override(prefill_layout=cols):
        kern.gdn_prefill_raw(pc, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yc, lens)
    for t in range(T):
        live = (t < lens).nonzero().flatten()
        yt = torch.empty(live.numel(), H, 128, device=DEV)
        kern.gdn_decode_raw(ps, slots[live].contiguous(), inp["q"][live, t].contiguous(),
                            inp["k"][live, t].contiguous(), inp["v"][live, t].contiguous(),
                            a[live, t].contiguous(), b[live, t].contiguous(), A, dtb, yt)
        assert torch.equal(yc[live, t], yt), f"token {t}: outputs differ"
        dead = (t >= lens).nonzero().flatten()
        assert bool((yc[dead, t] == 0).all()), f"token {t}: pad outputs are not 0"
    torch.cuda.synchronize()
    same = (pc == ps) | (pc.isnan() & ps.isnan())
    assert bool(same.all()), f"states differ by {(pc.float() - ps.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("dt", POOL_DTYPES, ids=POOL_IDS)
def test_a_plan_with_every_tier_is_decode_bit_for_bit(kern, dt):
    """A planned launch forced to use all four tiers (the longest row in the
    eighth layout, the next quarter, the next split, the rest whole; the
    prefill_plan knob, n8 * 2^20 + n4 * 2^10 + n2) equals decode applied token
    by token, bit for bit, with zeros at the pad outputs."""
    lens_l = [37, 29, 18, 11, 0]
    B, T, H, G = len(lens_l), max(lens_l), 32, 16
    inp = prefill_inputs(B, T, H=H, G=G, seed=81)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=82)
    lens = torch.tensor(lens_l, dtype=torch.int32, device=DEV)
    slots = torch.tensor([6, 2, 0, 4, 1], dtype=torch.int32, device=DEV)
    pc = pool(8, H=H, dtype=dt)
    ps = pc.clone()
    yc = torch.empty(B, T, H, 128, device=DEV)
    with kern.launch_override(prefill_layout=0, prefill_plan=(1 << 20) | (1 << 10) | 1):
        kern.gdn_prefill_raw(pc, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yc, lens)
    for t in range(T):
        live = (t < lens).nonzero().flatten()
        yt = torch.empty(live.numel(), H, 128, device=DEV)
        kern.gdn_decode_raw(ps, slots[live].contiguous(), inp["q"][live, t].contiguous(),
                            inp["k"][live, t].contiguous(), inp["v"][live, t].contiguous(),
                            a[live, t].contiguous(), b[live, t].contiguous(), A, dtb, yt)
        assert torch.equal(yc[live, t], yt), f"token {t}: outputs differ"
        dead = (t >= lens).nonzero().flatten()
        assert bool((yc[dead, t] == 0).all()), f"token {t}: pad outputs are not 0"
    torch.cuda.synchronize()
    same = (pc == ps) | (pc.isnan() & ps.isnan())
    assert bool(same.all()), f"states differ by {(pc.float() - ps.float()).abs().max().item():.3e}"


def test_a_skewed_ragged_batch_is_decode_bit_for_bit(kern):
    """One long row among short ones: the default launch plans the long row's
    tiles in the quarter layout (its chain, not the total work, bounds the
    batch) and the rest whole. Outputs and states must equal decode applied
    token by token, bit for bit, with zeros at the pad outputs."""
    lens_l = [256] + [32] * 15
    B, T, H, G = len(lens_l), max(lens_l), 32, 16
    inp = prefill_inputs(B, T, H=H, G=G, seed=31)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=32)
    lens = torch.tensor(lens_l, dtype=torch.int32, device=DEV)
    slots = torch.arange(3, B + 3, dtype=torch.int32, device=DEV)
    pc = pool(B + 4, H=H, dtype=torch.float16)
    ps = pc.clone()
    yc = torch.empty(B, T, H, 128, device=DEV)
    kern.gdn_prefill_raw(pc, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yc, lens)
    for t in range(T):
        live = (t < lens).nonzero().flatten()
        yt = torch.empty(live.numel(), H, 128, device=DEV)
        kern.gdn_decode_raw(ps, slots[live].contiguous(), inp["q"][live, t].contiguous(),
                            inp["k"][live, t].contiguous(), inp["v"][live, t].contiguous(),
                            a[live, t].contiguous(), b[live, t].contiguous(), A, dtb, yt)
        assert torch.equal(yc[live, t], yt), f"token {t}: outputs differ"
    assert bool((yc[1:, 32:] == 0).all()), "pad outputs are not 0"
    torch.cuda.synchronize()
    assert torch.equal(pc.view(torch.int16), ps.view(torch.int16))


def test_host_planned_eager_prefill_equals_the_captured_one(kern):
    """An eager ragged prefill runs the plan the host chooses from seq_lens; a
    captured one cannot read them and plans in the kernel. The plans differ
    (here the host runs the longest row in the quarter layout and five rows
    split), the bits may not: states and outputs are equal, and equal to
    decode applied token by token on a sampled row."""
    lens_l = [454, 610, 334, 542, 393, 861, 814, 65]
    B, T, H, G = len(lens_l), max(lens_l), 32, 16
    inp = prefill_inputs(B, T, H=H, G=G, seed=71)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=72)
    lens = torch.tensor(lens_l, dtype=torch.int32, device=DEV)
    slots = torch.arange(1, B + 1, dtype=torch.int32, device=DEV)
    base = pool(B + 2, H=H, dtype=torch.float16)
    pe, ye = base.clone(), torch.empty(B, T, H, 128, device=DEV)
    kern.gdn_prefill_raw(pe, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, ye, lens)
    pg, yg = base.clone(), torch.empty(B, T, H, 128, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        kern.gdn_prefill_raw(pg, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yg, lens)
    torch.cuda.current_stream().wait_stream(s)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(pe.view(torch.int16), pg.view(torch.int16)), "states differ"
    assert torch.equal(ye, yg), "outputs differ"
    # the 65-token row against decode token by token
    r = 7
    ps = base.clone()
    for t in range(lens_l[r]):
        yt = torch.empty(1, H, 128, device=DEV)
        kern.gdn_decode_raw(ps, slots[r:r + 1].contiguous(), inp["q"][r:r + 1, t].contiguous(),
                            inp["k"][r:r + 1, t].contiguous(), inp["v"][r:r + 1, t].contiguous(),
                            a[r:r + 1, t].contiguous(), b[r:r + 1, t].contiguous(), A, dtb, yt)
        assert torch.equal(yt[0], ye[r, t]), t
    torch.cuda.synchronize()
    assert torch.equal(ps[slots[r]].view(torch.int16), pe[slots[r]].view(torch.int16))


def test_a_captured_prefill_with_a_host_plan_equals_the_eager_one(kern):
    """Under capture the caller can hand the library the plan it would choose
    from host lengths (plan_lens). The graph keeps that plan; replayed over the
    lengths it was planned for and over other lengths, it leaves the eager
    prefill's bits, since every plan computes the same bits."""
    lens_l = [454, 610, 334, 542, 393, 861, 814, 65]
    B, T, H, G = len(lens_l), max(lens_l), 32, 16
    inp = prefill_inputs(B, T, H=H, G=G, seed=81)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=82)
    lens = torch.tensor(lens_l, dtype=torch.int32, device=DEV)
    slots = torch.arange(1, B + 1, dtype=torch.int32, device=DEV)
    base = pool(B + 2, H=H, dtype=torch.float16)
    assert kern.prefill_plan(lens_l, T, H) != 0  # a mixed plan, not all-whole
    pg, yg = base.clone(), torch.empty(B, T, H, 128, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        kern.gdn_prefill_raw(pg, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yg, lens,
                             plan_lens=lens_l)
    torch.cuda.current_stream().wait_stream(s)
    for replay_lens in (lens_l, [T, 1, 0, 300, 861, 2, 700, 64]):
        lens.copy_(torch.tensor(replay_lens, dtype=torch.int32))
        pe, ye = base.clone(), torch.empty(B, T, H, 128, device=DEV)
        kern.gdn_prefill_raw(pe, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, ye, lens)
        pg.copy_(base)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(pe.view(torch.int16), pg.view(torch.int16)), replay_lens
        assert torch.equal(ye, yg), replay_lens


def test_a_plan_needs_seq_lens(kern):
    B, T, H, G = 2, 8, 32, 16
    inp = prefill_inputs(B, T, H=H, G=G, seed=83)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=84)
    p = pool(4, H=H, dtype=torch.float16)
    y = torch.empty(B, T, H, 128, device=DEV)
    slots = torch.arange(B, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="seq_lens is required"):
        kern.gdn_prefill_raw(p, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, y,
                             plan_lens=[T, T])
