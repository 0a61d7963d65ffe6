"""The BASELINE configurations at full size, checked through size-independent
properties plus sampled-row oracle parity.

  config 1  batched decode B=128, 160-slot fp16 pool, random permutation of
            128 distinct slots, 64 consecutive steps
  config 2  ragged prefill, 8 sequences of U[64, 1024] tokens: native conv
            prefill + raw-gate chunk scan, bit-identical to conv1d_decode +
            gdn_decode_raw applied T_b times
  config 3  24 GDN layers of quant -> conv1d decode -> gated decode at B=64
  config 4  a mixed tick: 96 decode rows + 4 x 256-token prefill chunks on
            fresh slots of one 192-slot fp16 pool, eager and graph-captured
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from braid_amd.tick import MixedTick

import oracle
from gpu_helpers import (ATOL, DEV, RTOL, act_np, assert_parity, gen, to_np_pool, torch_gates,
                         ulp16)

pytestmark = pytest.mark.gpu
H, G, D, C = 32, 16, 128, 8192


def gate_consts(seed):
    g = gen(seed)
    A_log = torch.rand(H, generator=g, device=DEV) * 2
    dt_bias = torch.rand(H, generator=g, device=DEV) * 2 - 1
    return (-torch.exp(A_log)).contiguous(), dt_bias.contiguous()


def step_inputs(B, g, act=torch.bfloat16):
    return dict(
        q=torch.randn(B, G, D, generator=g, device=DEV),
        k=torch.randn(B, G, D, generator=g, device=DEV),
        v=torch.randn(B, H, D, generator=g, device=DEV),
        a=torch.randn(B, H, generator=g, device=DEV).to(act),
        b=torch.randn(B, H, generator=g, device=DEV).to(act),
    )


def oracle_decode_rows(ref_pool, slots, rows, inp, A, dtb, gates="oracle"):
    """The oracle's decode of `rows`. gates="torch": fed torch's gate
    spelling (gdn.py:299-300), which the in-kernel gates equal bit for bit,
    so the result is held to the max-abs bar; "oracle": the oracle's own
    gate restatement."""
    if gates == "torch":
        ta, tb = torch_gates(inp["a"][rows], inp["b"][rows], A, dtb)
        al, be = ta.cpu().numpy(), tb.cpu().numpy()
    else:
        al, be = oracle.gdn_gates(act_np(inp["a"][rows]), act_np(inp["b"][rows]),
                                  A.cpu().numpy(), dtb.cpu().numpy(), "bf16")
    return oracle.gdn_decode(ref_pool, slots, inp["q"][rows].cpu().numpy(),
                             inp["k"][rows].cpu().numpy(), inp["v"][rows].cpu().numpy(), al, be,
                             "f16")


def test_config1_batched_decode_b128_fp16_pool_64_steps(kern):
    B, S, steps = 128, 160, 64
    g = gen(1)
    pool = (torch.randn(S, H, D, D, generator=g, device=DEV) * 0.02).half().contiguous()
    perm = torch.randperm(S, generator=torch.Generator().manual_seed(1))
    slots = perm[:B].to(torch.int32).to(DEV)
    unused = perm[B:].tolist()
    before_unused = pool[unused].clone()
    A, dtb = gate_consts(2)
    y = torch.empty(B, H, D, device=DEV)
    rows = [0, 1, 37, 64, 100, 127]
    row_slots = slots[rows].long()
    local = np.arange(len(rows))
    worst_ulp, worst_y, worst_abs = 0, 0.0, 0.0
    for step in range(steps):
        inp = step_inputs(B, g)
        # teacher-forced: one oracle step from the kernel's current state, with
        # torch's gate spelling (bitwise the kernel's)
        ref_pool = to_np_pool(pool[row_slots])
        y_ref = oracle_decode_rows(ref_pool, local, rows, inp, A, dtb, gates="torch")
        kern.gdn_decode_raw(pool, slots, inp["q"], inp["k"], inp["v"], inp["a"], inp["b"], A,
                            dtb, y)
        d = ulp16(to_np_pool(pool[row_slots]), ref_pool)
        worst_ulp = max(worst_ulp, int(d.max()))
        yr = y[rows].cpu().numpy()
        err = np.abs(yr - y_ref) - (ATOL + RTOL * np.abs(y_ref))
        worst_y = max(worst_y, float(err.max()))
        worst_abs = max(worst_abs, float(np.abs(yr.astype(np.float64) - y_ref).max()))
    print(f"  config 1, 64 steps: y max-abs {worst_abs:.3e} (bar 2e-5), state within "
          f"{worst_ulp} fp16 ulp", flush=True)
    assert worst_abs <= 2e-5, f"y max-abs error {worst_abs:.3e} exceeds 2e-5"
    assert worst_ulp <= 1, f"state beyond one fp16 ulp of the oracle: {worst_ulp}"
    assert worst_y <= 0, f"y beyond tolerance by {worst_y:.3e}"
    assert torch.equal(pool[unused], before_unused), "an unused slot changed"
    assert torch.isfinite(pool.float()).all()


def test_config2_ragged_prefill_equals_decode_t_times(kern):
    """Config 2 end to end on the native kernels: causal conv prefill (fp16
    weights widened to fp32, SiLU) then the raw-gate chunk scan with seq_lens,
    against the decode path — conv1d_decode then gdn_decode_raw on strided
    q/k/v views — applied token by token. Conv windows, states and every live
    output must be bit-identical."""
    B = 8
    lens = torch.randint(64, 1025, (B,), generator=torch.Generator().manual_seed(2))
    T = int(lens.max())
    g = gen(3)
    w = (torch.randn(C, 4, generator=g, device=DEV) * 0.1).half().float()
    x = torch.randn(B, T, C, generator=g, device=DEV).to(torch.bfloat16)
    a_raw = torch.randn(B, T, H, generator=g, device=DEV)
    b_raw = torch.randn(B, T, H, generator=g, device=DEV)
    A, dtb = gate_consts(4)
    pool0 = (torch.randn(12, H, D, D, generator=g, device=DEV) * 0.02).half()
    conv0 = torch.zeros(12, C, 4, device=DEV)
    slots = torch.tensor([11, 3, 7, 0, 5, 9, 2, 6], dtype=torch.int32, device=DEV)
    seq = lens.to(torch.int32).to(DEV)

    # prefill path
    pc, cc = pool0.clone(), conv0.clone()
    qkv = torch.empty(B, T, C, device=DEV)
    kern.conv1d_prefill(cc, slots, x, w, None, qkv, seq)
    q = qkv[..., : G * D].reshape(B, T, G, D).contiguous()
    k = qkv[..., G * D: 2 * G * D].reshape(B, T, G, D).contiguous()
    v = qkv[..., 2 * G * D:].reshape(B, T, H, D).contiguous()
    yc = torch.empty(B, T, H, D, device=DEV)
    kern.gdn_prefill_raw(pc, slots, q, k, v, a_raw, b_raw, A, dtb, yc, seq)

    # decode path, one token at a time
    ps, cs = pool0.clone(), conv0.clone()
    lens_l = lens.tolist()
    for t in range(T):
        live = [b for b in range(B) if t < lens_l[b]]
        sl = slots[live].contiguous()
        co = torch.empty(len(live), C, device=DEV)
        kern.conv1d_decode(cs, sl, x[live, t].contiguous(), w, None, co)
        qd, kd, vd = torch.split(co, [G * D, G * D, H * D], dim=-1)
        ys = torch.empty(len(live), H, D, device=DEV)
        kern.gdn_decode_raw(ps, sl, qd.unflatten(-1, (G, D)), kd.unflatten(-1, (G, D)),
                            vd.unflatten(-1, (H, D)), a_raw[live, t].contiguous(),
                            b_raw[live, t].contiguous(), A, dtb, ys)
        assert torch.equal(co, qkv[live, t]), f"token {t}: conv outputs differ"
        assert torch.equal(ys, yc[live, t]), f"token {t}: scan outputs differ"
    assert torch.equal(cc, cs), "conv windows differ from decode applied T_b times"
    assert torch.equal(pc, ps), "final states differ from decode applied T_b times"
    untouched = [1, 4, 8, 10]
    assert torch.equal(pc[untouched], pool0[untouched])


def test_config3_mixer_decode_24_layers_b64(kern):
    B, layers = 64, 24
    g = gen(5)
    S = B + 8
    slots = torch.randperm(S, generator=torch.Generator().manual_seed(5))[:B].to(torch.int32).to(DEV)
    for layer in range(layers):
        x = torch.randn(B, 4096, generator=g, device=DEV, dtype=torch.bfloat16)
        xq, xs = kern.quantize_act(x)
        qo, so = oracle.quantize_act(x.float().cpu().numpy())
        assert xs.item() == float(so)
        assert np.array_equal(xq.view(torch.uint8).cpu().numpy(), qo), f"layer {layer}: fp8"
        if layer % 8:
            continue  # full conv/scan parity on layers 0, 8, 16 (all run above)
        conv_pool = torch.randn(S, C, 4, generator=g, device=DEV) * 0.5
        w = (torch.randn(C, 4, generator=g, device=DEV) * 0.1).half().float()
        bias = torch.randn(C, generator=g, device=DEV) * 0.1
        xin = torch.randn(B, C, generator=g, device=DEV, dtype=torch.bfloat16)
        ref_conv = conv_pool.cpu().numpy().copy()
        out_ref = oracle.conv1d_decode(ref_conv, slots.cpu().numpy(), xin.float().cpu().numpy(),
                                       w.cpu().numpy(), bias.cpu().numpy())
        conv_out = torch.empty(B, C, device=DEV)
        kern.conv1d_decode(conv_pool, slots, xin, w, bias, conv_out)
        np.testing.assert_allclose(conv_out.cpu().numpy(), out_ref, rtol=RTOL, atol=ATOL)
        q, k, v = torch.split(conv_out, [G * D, G * D, H * D], dim=-1)
        q, k, v = q.unflatten(-1, (G, D)), k.unflatten(-1, (G, D)), v.unflatten(-1, (H, D))
        pool = (torch.randn(S, H, D, D, generator=g, device=DEV) * 0.02).half()
        A, dtb = gate_consts(6 + layer)
        a = torch.randn(B, H, generator=g, device=DEV).to(torch.bfloat16)
        b = torch.randn(B, H, generator=g, device=DEV).to(torch.bfloat16)
        rows = [0, 17, 63]
        ref_pool = to_np_pool(pool)
        inp = dict(q=q, k=k, v=v, a=a, b=b)
        y_ref = oracle_decode_rows(ref_pool, slots[rows].cpu().numpy(), rows, inp, A, dtb,
                                   gates="torch")
        y = torch.empty(B, H, D, device=DEV)
        kern.gdn_decode_raw(pool, slots, q, k, v, a, b, A, dtb, y)
        assert_parity(y[rows].cpu().numpy(), y_ref, f"config 3 layer {layer} y")
        d = ulp16(to_np_pool(pool)[slots[rows].cpu().numpy()],
                  ref_pool[slots[rows].cpu().numpy()])
        assert d.max() <= 1


def test_config4_mixed_tick_eager_equals_graph_per_bucket(kern):
    S, n_dec, n_pre, T = 192, 96, 4, 256
    g = gen(7)
    pool0 = (torch.randn(S, H, D, D, generator=g, device=DEV) * 0.02).half()
    A, dtb = gate_consts(8)
    dec_slots = torch.arange(n_dec, dtype=torch.int32, device=DEV)
    pre_slots = torch.arange(n_dec, n_dec + n_pre, dtype=torch.int32, device=DEV)
    pool0[pre_slots.long()] = 0  # fresh slots
    scratch = S - 1
    dec = step_inputs(n_dec, g)
    pre = dict(q=torch.randn(n_pre, T, G, D, generator=g, device=DEV),
               k=torch.randn(n_pre, T, G, D, generator=g, device=DEV),
               v=torch.randn(n_pre, T, H, D, generator=g, device=DEV),
               a=torch.randn(n_pre, T, H, generator=g, device=DEV).to(torch.bfloat16),
               b=torch.randn(n_pre, T, H, generator=g, device=DEV).to(torch.bfloat16))
    seq = torch.full((n_pre,), T, dtype=torch.int32, device=DEV)

    # eager reference tick
    pe = pool0.clone()
    ye_pre = torch.empty(n_pre, T, H, D, device=DEV)
    kern.gdn_prefill_raw(pe, pre_slots, pre["q"], pre["k"], pre["v"], pre["a"], pre["b"], A, dtb,
                         ye_pre, seq)
    ye_dec = torch.empty(n_dec, H, D, device=DEV)
    kern.gdn_decode_raw(pe, dec_slots, dec["q"], dec["k"], dec["v"], dec["a"], dec["b"], A, dtb,
                        ye_dec)

    for bucket in (16, 32, 64, 96, 128):
        live = min(bucket, n_dec)
        pad = bucket - live
        sl = torch.cat([dec_slots[:live], torch.full((pad,), scratch, dtype=torch.int32,
                                                      device=DEV)])
        def padded(t):
            return torch.cat([t[:live], t[:1].expand(pad, *t.shape[1:])]).contiguous()
        bi = {k: padded(v) for k, v in dec.items()}
        pg = pool0.clone()
        y_pre = torch.empty(n_pre, T, H, D, device=DEV)
        y_dec = torch.empty(bucket, H, D, device=DEV)

        def tick_seq():
            kern.gdn_prefill_raw(pg, pre_slots, pre["q"], pre["k"], pre["v"], pre["a"],
                                 pre["b"], A, dtb, y_pre, seq)
            kern.gdn_decode_raw(pg, sl, bi["q"], bi["k"], bi["v"], bi["a"], bi["b"], A, dtb,
                                y_dec)

        # the same tick with the decode beside the prefill (MixedTick)
        side_by_side = MixedTick(kern, check_slots=True)
        pre_args = dict(slots=pre_slots, q=pre["q"], k=pre["k"], v=pre["v"], a_raw=pre["a"],
                        b_raw=pre["b"], A=A, dt_bias=dtb, y=y_pre, seq_lens=seq)
        dec_args = dict(slots=sl, q=bi["q"], k=bi["k"], v=bi["v"], a_raw=bi["a"],
                        b_raw=bi["b"], A=A, dt_bias=dtb, y=y_dec)

        def tick_mixed():
            side_by_side(pg, pre_args, dec_args)

        def check(label):
            assert torch.equal(y_pre, ye_pre), f"bucket {bucket} {label}: prefill outputs"
            assert torch.equal(y_dec[:live], ye_dec[:live]), \
                f"bucket {bucket} {label}: decode outputs"
            assert torch.equal(pg[pre_slots.long()], pe[pre_slots.long()]), label
            assert torch.equal(pg[dec_slots[:live].long()], pe[dec_slots[:live].long()]), label
            others = [s for s in range(S) if s >= live and s not in
                      (n_dec, n_dec + 1, n_dec + 2, n_dec + 3, scratch)]
            assert torch.equal(pg[others], pool0[others]), label

        for label, tick in (("sequential", tick_seq), ("side by side", tick_mixed)):
            graph = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            if pad == 0:
                pg.copy_(pool0)
                with torch.cuda.stream(side):
                    tick()  # eager (validation on: slots distinct)
                torch.cuda.current_stream().wait_stream(side)
                torch.cuda.synchronize()
                check(label + ", eager")
            with torch.cuda.graph(graph):
                tick()
            for _ in range(2):
                pg.copy_(pool0)
                graph.replay()
                torch.cuda.synchronize()
                check(label + ", graph")
