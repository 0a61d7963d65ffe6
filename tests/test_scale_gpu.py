"""The hot path at serving scale: batches and chunks well beyond the bench's.

The reference's kernel tests stop at a few rows and short chunks
(tests/test_gdn_decode_kernel.py, test_gdn_prefill_kernel.py:84-206); its
server decodes up to its max_batch rows a tick and prefills whole prompts.
At these sizes the oracle would take minutes, so the checks are the
size-independent ones: a batch equals the same rows decoded in pieces (each
tile is one workgroup's work, so the launch shape may not change a bit), a
chunk equals decode applied token by token, untouched slots keep their bits,
and sampled rows still match the oracle.
"""
from __future__ import annotations

import pytest
import torch

import oracle
from gpu_helpers import (DEV, KIND, assert_parity, assert_pool_close, decode_inputs, pool,
                         prefill_inputs, raw_gates, to_np_pool, torch_gates)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", [torch.float16, torch.float32], ids=["f16-pool", "f32-pool"])
def test_a_large_batch_equals_its_pieces_and_the_oracle(kern, dt):
    """B = 1024 rows of 32 heads (32,768 tiles, 8x the bench's batch) on a
    pool of 1,100 slots, the slots a random permutation: the whole batch in
    one launch leaves the same bits as the rows decoded in four launches of
    1, 127, 384 and 512 rows; the 76 slots no row names keep their bits; three
    sampled rows match the oracle."""
    B, H, G, S = 1024, 32, 16, 1100
    print(f"  large decode B={B} H={H} {KIND[dt]} pool of {S} slots", flush=True)
    slots = torch.randperm(S, generator=torch.Generator().manual_seed(5))[:B]
    slots = slots.to(torch.int32).to(DEV)
    inp = decode_inputs(B, H=H, G=G, seed=41)
    a_raw, b_raw, A, dt_bias = raw_gates((B, H), H, torch.bfloat16, seed=42)
    base = pool(S, H=H, dtype=dt, seed=43)
    pw = base.clone()
    yw = torch.empty(B, H, 128, device=DEV)
    kern.gdn_decode_raw(pw, slots, inp["q"], inp["k"], inp["v"], a_raw, b_raw, A, dt_bias, yw)
    pp = base.clone()
    yp = torch.empty(B, H, 128, device=DEV)
    lo = 0
    for n in (1, 127, 384, 512):
        r = slice(lo, lo + n)
        out = torch.empty(n, H, 128, device=DEV)
        kern.gdn_decode_raw(pp, slots[r].contiguous(), inp["q"][r].contiguous(),
                            inp["k"][r].contiguous(), inp["v"][r].contiguous(),
                            a_raw[r].contiguous(), b_raw[r].contiguous(), A, dt_bias, out)
        yp[r] = out
        lo += n
    torch.cuda.synchronize()
    assert torch.equal(yw, yp), "outputs differ between one launch and four"
    assert torch.equal(pw.view(torch.uint8), pp.view(torch.uint8)), "states differ"
    named = torch.zeros(S, dtype=torch.bool, device=DEV)
    named[slots.long()] = True
    free = (~named).nonzero().flatten()
    assert free.numel() == S - B
    assert torch.equal(pw[free].view(torch.uint8), base[free].view(torch.uint8)), \
        "a slot no row names changed"
    rows = [0, 613, B - 1]
    sub = slots[rows].long()
    ref_pool = to_np_pool(base[sub])
    alpha, beta = torch_gates(a_raw, b_raw, A, dt_bias)
    n_ = {k: v[rows].cpu().numpy() for k, v in inp.items()}
    y_ref = oracle.gdn_decode(ref_pool, [0, 1, 2], n_["q"], n_["k"], n_["v"],
                              alpha[rows].cpu().numpy(), beta[rows].cpu().numpy(), KIND[dt])
    assert_parity(yw[rows].cpu().numpy(), y_ref, "y of sampled rows")
    assert_pool_close(pw[sub].contiguous(), ref_pool, slice(0, 3), "sampled rows' states")


def test_a_long_ragged_chunk_equals_decode_applied_t_times(kern):
    """A 2,048-token chunk (the bench's prefill is 256 tokens a row) on an
    fp16 pool, two rows of 2,048 and 1,500 live tokens: every output and the
    final states equal decode applied token by token, bit for bit, and the
    pad outputs are zero."""
    B, T, H, G = 2, 2048, 32, 16
    print(f"  long prefill B={B} T={T} H={H} f16 pool", flush=True)
    inp = prefill_inputs(B, T, H=H, G=G, seed=51)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=52)
    lens_l = [2048, 1500]
    lens = torch.tensor(lens_l, dtype=torch.int32, device=DEV)
    slots = torch.tensor([3, 1], dtype=torch.int32, device=DEV)
    pc = pool(4, H=H, dtype=torch.float16, seed=53)
    ps = pc.clone()
    yc = torch.empty(B, T, H, 128, device=DEV)
    kern.gdn_prefill_raw(pc, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yc, lens)
    ys = torch.zeros(B, T, H, 128, device=DEV)
    for t in range(T):
        live = [r for r in range(B) if t < lens_l[r]]
        yt = torch.empty(len(live), H, 128, device=DEV)
        kern.gdn_decode_raw(ps, slots[live].contiguous(), inp["q"][live, t].contiguous(),
                            inp["k"][live, t].contiguous(), inp["v"][live, t].contiguous(),
                            a[live, t].contiguous(), b[live, t].contiguous(), A, dtb, yt)
        ys[live, t] = yt
    torch.cuda.synchronize()
    assert torch.equal(yc, ys), f"outputs differ by {(yc - ys).abs().max().item():.3e}"
    assert torch.equal(pc.view(torch.int16), ps.view(torch.int16)), "states differ"


def test_a_wide_ragged_prefill_equals_decode_applied_t_times(kern):
    """256 rows with lengths drawn from 0..96 (a serving tick's worth of new
    prompts, ragged, some empty), the host planning the launch: outputs and
    states equal decode applied token by token, bit for bit."""
    B, T, H, G = 256, 96, 32, 16
    print(f"  wide ragged prefill B={B} T<={T} H={H} bf16 pool", flush=True)
    g = torch.Generator().manual_seed(61)
    lens_l = torch.randint(0, T + 1, (B,), generator=g).tolist()
    lens_l[7] = T
    lens_l[8] = 0
    inp = prefill_inputs(B, T, H=H, G=G, seed=62)
    a, b, A, dtb = raw_gates((B, T, H), H, torch.bfloat16, seed=63)
    lens = torch.tensor(lens_l, dtype=torch.int32, device=DEV)
    slots = torch.randperm(B + 8, generator=g)[:B].to(torch.int32).to(DEV)
    pc = pool(B + 8, H=H, dtype=torch.bfloat16, seed=64)
    ps = pc.clone()
    yc = torch.empty(B, T, H, 128, device=DEV)
    kern.gdn_prefill_raw(pc, slots, inp["q"], inp["k"], inp["v"], a, b, A, dtb, yc, lens)
    ys = torch.zeros(B, T, H, 128, device=DEV)
    for t in range(T):
        live = [r for r in range(B) if t < lens_l[r]]
        if not live:
            continue
        li = torch.tensor(live, device=DEV)
        yt = torch.empty(len(live), H, 128, device=DEV)
        kern.gdn_decode_raw(ps, slots[li].contiguous(), inp["q"][li, t].contiguous(),
                            inp["k"][li, t].contiguous(), inp["v"][li, t].contiguous(),
                            a[li, t].contiguous(), b[li, t].contiguous(), A, dtb, yt)
        ys[li, t] = yt
    torch.cuda.synchronize()
    assert torch.equal(yc, ys), f"outputs differ by {(yc - ys).abs().max().item():.3e}"
    assert torch.equal(pc.view(torch.int16), ps.view(torch.int16)), "states differ"
