"""Pins the CPU oracle (oracle/gdn_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible slip in the oracle — a dropped term,
decaying before reducing, a tiled instead of grouped head map, a missing
epsilon, the wrong softplus branch, an fp8 rounding or tie error — fails at
least one of them:
  * brute-force Python loops and a float64 closed form (tests/refmath.py);
  * the reference's invariants (tests/test_gdn_ref.py:54-97 of the reference:
    beta = 0 is pure decay, rows are independent, heads map to groups grouped);
  * the pad identity and chunk-split invariance (test_gdn_prefill_kernel.py);
  * committed golden fixtures from float64 math and torch's CPU spellings.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from braid_amd.config import GDNConfig
from refmath import (ACT_DTYPES, act_storage, check_readout, conv_f64, decode_f64, decode_naive,
                     e4m3_table, gates_f64, torch_gated_readout)

GOLDEN = Path(__file__).resolve().parent / "golden"


def _inputs(B, H, G, SS, HD, seed=0, state_scale=1.0):
    rng = np.random.default_rng(seed)
    return dict(
        state=(rng.standard_normal((B, H, SS, HD)) * state_scale).astype(np.float32),
        q=rng.standard_normal((B, G, SS)).astype(np.float32),
        k=rng.standard_normal((B, G, SS)).astype(np.float32),
        v=rng.standard_normal((B, H, HD)).astype(np.float32),
        alpha=(rng.random((B, H)) * 0.5 + 0.5).astype(np.float32),
        beta=rng.random((B, H)).astype(np.float32),
    )


def _run(d):
    st = d["state"].copy()
    y = oracle.gdn_decode_rows(st, d["q"], d["k"], d["v"], d["alpha"], d["beta"])
    return y, st


# --- the recurrence -----------------------------------------------------------

def test_oracle_matches_brute_force_loops():
    d = _inputs(3, 4, 2, 8, 8, seed=1)
    y, st = _run(d)
    y_n, st_n = decode_naive(d["state"], d["q"], d["k"], d["v"], d["alpha"], d["beta"])
    np.testing.assert_allclose(y, y_n, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(st, st_n, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("B", [1, 3])
def test_oracle_matches_float64_at_full_shape(B):
    d = _inputs(B, 32, 16, 128, 128, seed=2 + B, state_scale=0.02)
    y, st = _run(d)
    y64, st64 = decode_f64(d["state"], d["q"], d["k"], d["v"], d["alpha"], d["beta"])
    np.testing.assert_allclose(y, y64, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(st, st64, rtol=2e-5, atol=2e-6)


def test_oracle_matches_golden_decode_fixture():
    g = np.load(GOLDEN / "decode_f64.npz")
    st = g["state"].copy()
    y = oracle.gdn_decode_rows(st, g["q"], g["k"], g["v"], g["alpha"], g["beta"])
    np.testing.assert_allclose(y, g["y"], rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(st, g["state_out"], rtol=2e-5, atol=2e-6)


def test_zero_beta_is_pure_decay_bitwise():
    d = _inputs(1, 2, 1, 16, 16, seed=3)
    d["beta"][:] = 0
    before = d["state"].copy()
    _, st = _run(d)
    assert np.array_equal(st, before * d["alpha"][0, :, None, None])


def test_pad_step_is_an_exact_identity():
    d = _inputs(2, 4, 2, 128, 128, seed=4)
    d["alpha"][:] = 1
    d["beta"][:] = 0
    _, st = _run(d)
    assert np.array_equal(st, d["state"])


def test_rows_are_independent_bitwise():
    d = _inputs(2, 4, 2, 32, 32, seed=5)
    solo = {k: v[1:2].copy() for k, v in d.items()}
    y2, st2 = _run(d)
    y1, st1 = _run(solo)
    assert np.array_equal(y2[1:2], y1) and np.array_equal(st2[1:2], st1)


def test_heads_map_to_groups_grouped_not_tiled():
    d = _inputs(1, 4, 2, 8, 8, seed=6)
    base = {k: v.copy() for k, v in d.items()}
    d["q"][:, 1] = 0
    d["k"][:, 1] = 0
    y_z, _ = _run(d)
    y_b, _ = _run(base)
    same = [bool(np.allclose(y_z[0, h], y_b[0, h])) for h in range(4)]
    assert same == [True, True, False, False]


def test_kv_uses_the_undecayed_state():
    """delta = (v - alpha * kv) * beta with kv on S, not on alpha*S: at alpha=0.5,
    the two readings differ by a factor on kv that float64 distinguishes."""
    d = _inputs(1, 2, 1, 16, 16, seed=7)
    d["alpha"][:] = 0.5
    y, _ = _run(d)
    y64, _ = decode_f64(d["state"], d["q"], d["k"], d["v"], d["alpha"], d["beta"])
    np.testing.assert_allclose(y, y64, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kind", ["f32", "f16", "bf16"])
def test_prefill_is_decode_applied_t_times_and_chunks_compose(kind):
    rng = np.random.default_rng(8)
    B, T, H, G = 2, 6, 4, 2
    q = rng.standard_normal((B, T, G, 128)).astype(np.float32)
    k = rng.standard_normal((B, T, G, 128)).astype(np.float32)
    v = rng.standard_normal((B, T, H, 128)).astype(np.float32)
    alpha = rng.uniform(0.5, 1, (B, T, H)).astype(np.float32)
    beta = rng.uniform(0, 1, (B, T, H)).astype(np.float32)
    pool0 = oracle.narrow(rng.standard_normal((5, H, 128, 128)).astype(np.float32) * 0.1, kind)
    slots = np.array([3, 1])
    p_chunk = pool0.copy()
    y_chunk = oracle.gdn_prefill(p_chunk, slots, q, k, v, alpha, beta, kind)
    p_step = pool0.copy()
    for t in range(T):
        y_t = oracle.gdn_decode(p_step, slots, q[:, t], k[:, t], v[:, t], alpha[:, t],
                                beta[:, t], kind)
        assert np.array_equal(y_t, y_chunk[:, t])
    assert np.array_equal(p_chunk, p_step)
    p_two = pool0.copy()
    oracle.gdn_prefill(p_two, slots, q[:, :2], k[:, :2], v[:, :2], alpha[:, :2], beta[:, :2], kind)
    oracle.gdn_prefill(p_two, slots, q[:, 2:], k[:, 2:], v[:, 2:], alpha[:, 2:], beta[:, 2:], kind)
    assert np.array_equal(p_two, p_chunk)
    untouched = [0, 2, 4]
    assert np.array_equal(p_chunk[untouched], pool0[untouched])


# --- storage emulation ----------------------------------------------------------

def test_narrowing_matches_torch_casts():
    rng = np.random.default_rng(9)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 3,
                        np.array([0.0, -0.0, 65504, 65520, 1e-8, np.inf, -np.inf],
                                 dtype=np.float32)])
    t = torch.from_numpy(x)
    assert np.array_equal(oracle.narrow(x, "f16").view(np.uint16),
                          t.half().numpy().view(np.uint16))
    assert np.array_equal(oracle.narrow(x, "bf16"), t.bfloat16().view(torch.uint16).numpy())
    assert oracle.narrow(np.array([np.nan], np.float32), "bf16")[0] == 0x7FC0


# --- gates --------------------------------------------------------------------------

@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_gates_match_torch_cpu_spelling_fixture(act):
    g = np.load(GOLDEN / "gates_torch.npz")
    a, b = g[f"a_{act}"], g[f"b_{act}"]
    if act == "bf16":
        a, b = oracle.bf16_bits(a), oracle.bf16_bits(b)
    alpha, beta = oracle.gdn_gates(a, b, g["A"], g["dt_bias"], act)
    # torch's CPU exp/log1p (vectorised) and libm agree to an ulp or two in
    # the exponent z = A * sp, which exp turns into a relative error ~ |z| ulp.
    with np.errstate(divide="ignore"):
        np.testing.assert_allclose(np.log(alpha), np.log(g[f"alpha_{act}"]), rtol=4e-7,
                                   atol=2e-7)
    if act == "f32":
        np.testing.assert_allclose(beta, g["beta_f32"], rtol=5e-7, atol=0)
    else:
        # rounded through bf16: equal except where an ulp-level fp32 difference
        # straddles a bf16 rounding boundary (then one bf16 ulp apart).
        diff = np.abs(beta - g["beta_bf16"])
        assert (diff <= np.abs(g["beta_bf16"]) * 2 ** -7).all()
        assert (diff == 0).mean() > 0.99
        assert np.array_equal(oracle.narrow(beta, "bf16"), oracle.bf16_bits(beta))


def test_gates_match_float64_and_take_the_threshold_branch():
    rng = np.random.default_rng(10)
    H = 32
    a = (rng.standard_normal((8, H)) * 4).astype(np.float32)
    probes = np.array([-80, -20, 0, 19, 19.999999, 20, 20.000001, 25, 80], np.float32)
    a[0, : probes.size] = probes
    b = (rng.standard_normal((8, H)) * 4).astype(np.float32)
    A = -np.exp(rng.uniform(0, 2, H)).astype(np.float32)
    dtb = np.zeros(H, np.float32)
    alpha, beta = oracle.gdn_gates(a, b, A, dtb, "f32")
    a64, b64 = gates_f64(a, b, A, dtb)
    live = a64 > 1e-30  # below that fp32 alpha underflows (to zero or a subnormal)
    np.testing.assert_allclose(np.log(alpha[live]), np.log(a64[live]), rtol=4e-7, atol=2e-7)
    assert (alpha[~live] < 1e-29).all()
    np.testing.assert_allclose(beta, b64, rtol=2e-6)
    # x > 20 takes sp = x exactly: alpha = fl(exp(fl(A * x)))
    for j in (6, 7, 8):
        x = np.float32(a[0, j])
        assert alpha[0, j] == np.float32(np.exp(np.float64(np.float32(A[j] * x))))


def test_seq_lens_pad_columns_and_edge_lengths():
    rng = np.random.default_rng(11)
    B, T, H = 3, 5, 4
    a = rng.standard_normal((B, T, H)).astype(np.float32)
    b = rng.standard_normal((B, T, H)).astype(np.float32)
    A = -np.ones(H, np.float32)
    dtb = np.zeros(H, np.float32)
    lens = np.array([0, 2, T + 3], np.int32)
    al, be = oracle.gdn_gates(a, b, A, dtb, "f32", seq_lens=lens)
    al0, be0 = oracle.gdn_gates(a, b, A, dtb, "f32")
    assert (al[0] == 1).all() and (be[0] == 0).all()
    assert (al[1, 2:] == 1).all() and (be[1, 2:] == 0).all()
    assert np.array_equal(al[1, :2], al0[1, :2]) and np.array_equal(al[2], al0[2])


# --- conv ---------------------------------------------------------------------------

def test_conv_matches_golden_fixture():
    g = np.load(GOLDEN / "conv_f64.npz")
    pool = g["window"].copy()
    out = oracle.conv1d_decode(pool, np.arange(pool.shape[0]), g["x"], g["weight"], g["bias"])
    np.testing.assert_allclose(out, g["out"], rtol=2e-5, atol=2e-6)
    np.testing.assert_array_equal(pool, g["window_out"])


def test_conv_silu_on_every_channel_known_answer():
    cfg = GDNConfig.qwen36_35b_a3b()
    C, K = cfg.conv_channels, cfg.conv_kernel
    assert C == 8192 and K == 4
    pool = np.zeros((2, C, K), np.float32)
    w = np.zeros((C, K), np.float32)
    w[:, -1] = 1
    out = oracle.conv1d_decode(pool, [0], np.full((1, C), -6.0, np.float32), w,
                               np.zeros(C, np.float32))
    expected = -6.0 / (1.0 + np.exp(6.0))
    np.testing.assert_allclose(out, expected, rtol=1e-6)


def test_conv_eight_rotating_steps_follow_the_slot():
    rng = np.random.default_rng(12)
    C, K, B, S = 64, 4, 4, 16
    pool = rng.standard_normal((S, C, K)).astype(np.float32)
    ref = pool.astype(np.float64)
    w = rng.standard_normal((C, K)).astype(np.float32)
    bias = rng.standard_normal(C).astype(np.float32)
    for step in range(8):
        slots = np.array([(step * 3 + i) % S for i in range(B)])
        x = rng.standard_normal((B, C)).astype(np.float32)
        out = oracle.conv1d_decode(pool, slots, x, w, bias)
        o64, win = conv_f64(ref[slots], x, w, bias)
        ref[slots] = win
        np.testing.assert_allclose(out, o64, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(pool, ref, rtol=0, atol=0)


# --- fp8 ----------------------------------------------------------------------------

def test_e4m3fn_matches_torch_cast_fixture():
    g = np.load(GOLDEN / "e4m3fn_torch.npz")
    assert np.array_equal(oracle.e4m3fn(g["x"]), g["codes"])


def test_e4m3fn_codes_round_trip_and_midpoints_go_to_even():
    vals = e4m3_table()
    codes = np.arange(0x7F)
    assert np.array_equal(oracle.e4m3fn(vals.astype(np.float32)), codes)
    assert np.array_equal(oracle.e4m3fn(-vals.astype(np.float32)), codes | 0x80)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    assert np.array_equal(oracle.e4m3fn(mids), np.where(codes[:-1] % 2 == 0, codes[:-1],
                                                        codes[:-1] + 1))
    assert oracle.e4m3fn(np.array([464.0, 464.5, 1e6, np.nan], np.float32)).tolist() == \
        [0x7E, 0x7F, 0x7F, 0x7F]


def test_quantize_act_scale_spelling_and_torch_codes():
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((8, 512)) * 3.5).astype(np.float32)
    q, sc = oracle.quantize_act(x)
    amax = np.float32(np.abs(x).max())
    assert sc == np.float32(amax * np.float32(1.0 / 448.0))
    ref = (torch.from_numpy(x) / torch.tensor(sc)).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert np.array_equal(q, ref.view(torch.uint8).numpy())


def test_quantize_act_degenerate_inputs():
    q, sc = oracle.quantize_act(np.zeros((4, 64), np.float32))
    assert sc == np.float32(1e-12) and (q == 0).all()
    q, sc = oracle.quantize_act(np.full((4, 64), 1e-10, np.float32))
    assert sc == np.float32(1e-12)
    assert (q == oracle.e4m3fn(np.array([np.float32(1e-10) / np.float32(1e-12)])) [0]).all()
    x = np.full((2, 64), 60000.0, np.float32)
    x[1] = -60000.0
    q, sc = oracle.quantize_act(x)
    assert (q[0] == 0x7E).all() and (q[1] == 0xFE).all()
    x = np.ones((4, 64), np.float32)
    x[2, 10] = np.nan
    q, sc = oracle.quantize_act(x)
    assert np.isnan(sc) and (q == 0x7F).all()


def test_state_bytes_match_reference_measurement():
    """63.75 MiB of recurrent state per sequence (reference test_gdn_ref.py:24-34)."""
    cfg = GDNConfig.qwen36_35b_a3b()
    assert abs(cfg.recurrent_bytes_per_seq / 2 ** 20 - 63.75) < 0.1


def test_conv_prefill_matches_the_reference_torch_spelling():
    """oracle.conv1d_prefill against the reference's own prefill conv, restated
    in torch on the CPU from braid/model/gdn.py:193-222: F.conv1d over
    [cached window | x] with no padding, the last T outputs, and the window
    saved by gathering joined[len : len + K] for a ragged row."""
    rng = np.random.default_rng(14)
    B, T, C, K = 3, 9, 32, 4
    pool = rng.standard_normal((5, C, K)).astype(np.float32)
    x = rng.standard_normal((B, T, C)).astype(np.float32)
    w = rng.standard_normal((C, K)).astype(np.float32)
    bias = rng.standard_normal(C).astype(np.float32)
    slots = np.array([3, 0, 4])
    lens = np.array([9, 4, 1])
    tp = torch.from_numpy(pool.copy())
    window = tp[torch.from_numpy(slots)]                                  # [B, C, K]
    joined = torch.cat([window, torch.from_numpy(x).transpose(1, 2)], -1)  # [B, C, K+T]
    idx = torch.from_numpy(lens)[:, None] + torch.arange(K)[None]
    keep = joined.gather(2, idx[:, None].expand(B, C, K))
    ref_out = F.silu(F.conv1d(joined, torch.from_numpy(w)[:, None, :], torch.from_numpy(bias),
                              padding=0, groups=C)[:, :, -T:]).transpose(1, 2).numpy()
    got_pool = pool.copy()
    out = oracle.conv1d_prefill(got_pool, slots, x, w, bias, lens)
    for b in range(B):
        np.testing.assert_allclose(out[b, :lens[b]], ref_out[b, :lens[b]], rtol=1e-5, atol=1e-6)
        assert (out[b, lens[b]:] == 0).all()
        np.testing.assert_array_equal(got_pool[slots[b]], keep[b].numpy())


# ---- gated RMSNorm readout ---------------------------------------------------

@pytest.mark.parametrize("act", ["bf16", "f16", "f32"])
def test_gated_rmsnorm_matches_torch_cpu_spelling(act):
    """Pins oracle.gated_rmsnorm to torch's own spelling of the readout: a
    dropped intermediate rounding, gamma applied before the cast, a sum
    instead of a mean or a sigmoid instead of silu moves far more than the
    handful of one-ulp ties that a different fp32 reduction order can flip."""
    rng = np.random.default_rng(21)
    N, H, HD = 48, 32, 128
    y = (rng.standard_normal((N, H, HD)) * 0.05).astype(np.float32)
    gamma = (1.0 + 0.3 * rng.standard_normal(HD)).astype(np.float32)
    zt = torch.from_numpy((rng.standard_normal((N, H, HD)) * 2).astype(np.float32)).to(ACT_DTYPES[act])
    eps = 1e-6
    ref = act_storage(torch_gated_readout(y, zt, gamma, eps, ACT_DTYPES[act]), act)
    got = oracle.gated_rmsnorm(y, act_storage(zt, act), gamma, eps, act)
    check_readout(got, ref, act)


def test_gated_rmsnorm_known_answer_one_hot_row():
    """y = [2, 0, ..., 0]: mean(c^2) = 4/128, so xf[0] = 2 * sqrt(32) = 11.3137
    -> bf16 11.3125; with gamma = 1 and z = 30 (silu(30) == 30 in fp32) the
    output is 339.375 -> bf16 340; every other element is exactly 0."""
    y = np.zeros((1, 128), np.float32)
    y[0, 0] = 2.0
    z = oracle.narrow(np.full((1, 128), 30.0, np.float32), "bf16")
    core = oracle.widen(oracle.gated_rmsnorm(y, z, np.ones(128, np.float32), 0.0, "bf16"), "bf16")
    assert core[0, 0] == np.float32(340.0)
    assert (core[0, 1:] == 0).all()


def test_gated_rmsnorm_scale_invariance_and_gate_limits():
    """With eps = 0 the norm is exactly invariant under a power-of-two scale
    of y (every rounding scales with it); silu(0) = 0 zeroes a unit; a
    negative gate flips the sign relative to silu's own sign."""
    rng = np.random.default_rng(22)
    y = rng.standard_normal((16, 128)).astype(np.float32)
    z = oracle.narrow(rng.standard_normal((16, 128)).astype(np.float32), "bf16")
    gamma = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    a = oracle.gated_rmsnorm(y, z, gamma, 0.0, "bf16")
    b = oracle.gated_rmsnorm(y * np.float32(64.0), z, gamma, 0.0, "bf16")
    assert np.array_equal(a, b)
    zero = oracle.narrow(np.zeros((16, 128), np.float32), "bf16")
    assert (oracle.widen(oracle.gated_rmsnorm(y, zero, gamma, 1e-6, "bf16"), "bf16") == 0).all()
    core = oracle.widen(a, "bf16")
    zf = oracle.widen(z, "bf16")
    nz = core != 0
    assert (np.sign(core[nz]) == np.sign(y[nz] * zf[nz])).all()


def test_torch_cpu_restatement_matches_the_c_oracle():
    """oracle/torch_ref.py (the CPU baseline bench.py times) restates the
    reference's batched torch step; it must agree with the pinned C oracle to
    the recurrence tolerance, state and outputs, on an fp16 pool with raw bf16
    gates."""
    import torch

    from oracle import torch_ref

    rng = np.random.default_rng(5)
    B, H, G, D, S = 3, 32, 16, 128, 6
    pool32 = (rng.standard_normal((S, H, D, D)) * 0.02).astype(np.float32)
    pool16 = pool32.astype(np.float16)
    slots = np.array([4, 0, 2], dtype=np.int32)
    q = rng.standard_normal((B, G, D)).astype(np.float32)
    k = rng.standard_normal((B, G, D)).astype(np.float32)
    v = rng.standard_normal((B, H, D)).astype(np.float32)
    a = oracle.bf16_bits(rng.standard_normal((B, H)).astype(np.float32))
    b = oracle.bf16_bits(rng.standard_normal((B, H)).astype(np.float32))
    A = -np.exp(rng.uniform(0, 2, H)).astype(np.float32)
    dtb = rng.uniform(-1, 1, H).astype(np.float32)

    al, be = oracle.gdn_gates(a, b, A, dtb, "bf16")
    ref_pool = pool16.copy()
    y_ref = oracle.gdn_decode(ref_pool, slots, q, k, v, al, be, "f16")

    tp = torch.from_numpy(pool16.copy())
    to_bf16 = lambda bits: torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)
    y = torch_ref.decode_step(tp, torch.from_numpy(slots), torch.from_numpy(q),
                              torch.from_numpy(k), torch.from_numpy(v), to_bf16(a), to_bf16(b),
                              torch.from_numpy(A), torch.from_numpy(dtb))
    np.testing.assert_allclose(y.numpy(), y_ref, rtol=2e-5, atol=2e-6)
    ulp = np.abs(tp.numpy().view(np.int16).astype(np.int32)
                 - ref_pool.view(np.int16).astype(np.int32))
    assert ulp.max() <= 1
    untouched = [1, 3, 5]
    assert np.array_equal(tp.numpy()[untouched], pool16[untouched])
