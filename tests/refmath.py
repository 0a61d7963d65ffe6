"""Independent float64 restatements used to pin the oracle (and the kernels).

These are written from the mathematics of the recurrence, not from the
oracle's C code: a brute-force triple loop over Python floats (the shape of
braid/reference/gdn_ref.py:42-66) and a vectorised float64 numpy closed form
(the shape of gdn_ref.py:69-99). Both take raw q/k and l2-normalise with the
additive epsilon, as the kernels do (gdn_decode.cu:213-227).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

L2_EPS = 1e-6


def l2norm64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + L2_EPS)


def decode_f64(state, q, k, v, alpha, beta):
    """float64 closed form. state [B,H,SS,HD] (returned updated copy), q,k
    [B,G,SS] raw, v [B,H,HD], alpha/beta [B,H]. Returns (y, state')."""
    S = np.array(state, dtype=np.float64)
    B, H, SS, HD = S.shape
    G = q.shape[1]
    hpg = H // G
    qh = np.repeat(l2norm64(q), hpg, axis=1)       # grouped: head h reads g = h // hpg
    kh = np.repeat(l2norm64(k), hpg, axis=1)
    a = np.asarray(alpha, np.float64)[..., None]
    b = np.asarray(beta, np.float64)[..., None]
    kv = np.einsum("bhsd,bhs->bhd", S, kh)
    delta = (np.asarray(v, np.float64) - a * kv) * b
    S = S * a[..., None] + kh[..., None] * delta[:, :, None, :]
    y = np.einsum("bhsd,bhs->bhd", S, qh) * HD ** -0.5
    return y, S


def decode_naive(state, q, k, v, alpha, beta):
    """Brute-force Python-float loops; tiny shapes only."""
    S = [[[[float(state[b, h, s, d]) for d in range(state.shape[3])]
           for s in range(state.shape[2])] for h in range(state.shape[1])]
         for b in range(state.shape[0])]
    B, H, SS, HD = state.shape
    G = q.shape[1]
    hpg = H // G
    y = np.zeros((B, H, HD))
    for b in range(B):
        for h in range(H):
            g = h // hpg
            qn = math.sqrt(sum(float(x) ** 2 for x in q[b, g]) + L2_EPS)
            kn = math.sqrt(sum(float(x) ** 2 for x in k[b, g]) + L2_EPS)
            qh = [float(x) / qn for x in q[b, g]]
            kh = [float(x) / kn for x in k[b, g]]
            a, bt = float(alpha[b, h]), float(beta[b, h])
            for d in range(HD):
                kv = sum(S[b][h][s][d] * kh[s] for s in range(SS))
                delta = (float(v[b, h, d]) - a * kv) * bt
                acc = 0.0
                for s in range(SS):
                    S[b][h][s][d] = a * S[b][h][s][d] + kh[s] * delta
                    acc += S[b][h][s][d] * qh[s]
                y[b, h, d] = acc / math.sqrt(HD)
    return y, np.array(S)


def gates_f64(a_raw, b_raw, A, dt_bias):
    """alpha = exp(A * softplus(a + dt_bias)), beta = sigmoid(b), float64."""
    x = np.asarray(a_raw, np.float64) + np.asarray(dt_bias, np.float64)
    sp = np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))
    alpha = np.exp(np.asarray(A, np.float64) * sp)
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b_raw, np.float64)))
    return alpha, beta


def conv_f64(window, x, weight, bias):
    """window [B,C,K] (returned slid copy), x [B,C] -> SiLU(sum w*W + bias)."""
    w = np.concatenate([np.asarray(window, np.float64)[:, :, 1:],
                        np.asarray(x, np.float64)[:, :, None]], axis=-1)
    acc = (w * np.asarray(weight, np.float64)[None]).sum(-1)
    if bias is not None:
        acc = acc + np.asarray(bias, np.float64)[None]
    return acc / (1.0 + np.exp(-acc)), w


def e4m3_table() -> np.ndarray:
    """Values of the 127 non-negative finite e4m3fn codes, from the format
    definition (bias 7, 3 mantissa bits, subnormals at exponent field 0)."""
    vals = []
    for code in range(0x7F):
        e, m = code >> 3, code & 7
        vals.append(m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    return np.array(vals)


def torch_gated_readout(y, z, gamma, eps, dtype):
    """The reference's readout restated in torch (CPU): braid/model/gdn.py:383-386
    casts the scan output to the activation dtype, then braid/model/norm.py:67-71
    normalises in fp32, rounds, applies gamma, gates with silu(z) in fp32 and
    rounds again."""
    x = (torch.from_numpy(y) if isinstance(y, np.ndarray) else y).to(dtype)
    g = torch.from_numpy(gamma) if isinstance(gamma, np.ndarray) else gamma
    gate = z
    xf = F.rms_norm(x.float(), (x.shape[-1],), None, eps)
    h = g.to(xf.device) * xf.to(dtype)
    h = h * F.silu(gate.float())
    return h.to(dtype)


ACT_DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def act_storage(t: torch.Tensor, act: str) -> np.ndarray:
    """Host copy of an act-dtype tensor in the oracle's storage convention."""
    t = t.detach().cpu()
    if act == "bf16":
        return t.view(torch.uint16).numpy()
    return t.numpy()


def act_ulps(a_bits, b_bits, act):
    """Distance in units in the last place between two arrays in act storage."""
    if act == "f32":
        ai = np.asarray(a_bits, np.float32).view(np.int32).astype(np.int64)
        bi = np.asarray(b_bits, np.float32).view(np.int32).astype(np.int64)
    else:
        ai = np.asarray(a_bits).view(np.int16).astype(np.int64)
        bi = np.asarray(b_bits).view(np.int16).astype(np.int64)
    # sign-magnitude -> ordered integers
    bits = 31 if act == "f32" else 15
    ai = np.where(ai < 0, -(ai & ((1 << bits) - 1)), ai)
    bi = np.where(bi < 0, -(bi & ((1 << bits) - 1)), bi)
    return np.abs(ai - bi)


# Tolerance of the gated readout against torch's spelling or the oracle, in
# ulps of the act dtype. The two differ only in the fp32 rounding of the
# reduction and rsqrt (and the last bits of exp); for 16-bit activations that
# can flip the rounding of xf.to(act), a change of up to 2^-7 relative, which
# moves the exact output by up to two of its own ulps before its rounding
# (three after it). Such flips are rare, so at least 99.5% of elements must be
# bit-identical. fp32 activations have no intermediate rounding: 8 ulps, 1e-6
# relative.
READOUT_ULPS = {"bf16": 3, "f16": 3, "f32": 8}


def check_readout(got_bits, ref_bits, act, label=""):
    u = act_ulps(got_bits, ref_bits, act)
    assert u.max() <= READOUT_ULPS[act], (label, int(u.max()))
    if act != "f32":
        assert (u == 0).mean() >= 0.995, (label, float((u == 0).mean()))
        assert (u > 1).mean() <= 1e-4, (label, float((u > 1).mean()))
