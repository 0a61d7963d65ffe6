"""Writes the committed golden fixtures in this folder.

None of the fixtures comes from running the reference: its kernels are CUDA
and its Python oracle is pinned here by independent computations instead.
The expected outputs are produced by
  * float64 closed forms written from the mathematics (tests/refmath.py), and
  * PyTorch's own CPU spellings (the third-party arithmetic the reference's
    bit-specs defer to: torch.sigmoid / F.softplus / torch.exp for the gates,
    gdn.py:299-300, and Tensor.to(torch.float8_e4m3fn) for the fp8 codes,
    quant.py:115,228-229).

Run:  python tests/golden/make_golden.py   (deterministic; seeds fixed)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from refmath import conv_f64, decode_f64  # noqa: E402


def decode_fixture():
    rng = np.random.default_rng(1234)
    B, H, G, D = 1, 2, 1, 128
    state = (rng.standard_normal((B, H, D, D)) * 0.02).astype(np.float32)
    q = rng.standard_normal((B, G, D)).astype(np.float32)
    k = rng.standard_normal((B, G, D)).astype(np.float32)
    v = rng.standard_normal((B, H, D)).astype(np.float32)
    alpha = rng.uniform(0.5, 1.0, (B, H)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (B, H)).astype(np.float32)
    y, s = decode_f64(state, q, k, v, alpha, beta)
    np.savez_compressed(HERE / "decode_f64.npz", state=state, q=q, k=k, v=v, alpha=alpha,
                        beta=beta, y=y.astype(np.float32), state_out=s.astype(np.float32))


def gates_fixture():
    g = torch.Generator().manual_seed(77)
    H = 32
    a32 = torch.randn(4, H, generator=g) * 3
    b32 = torch.randn(4, H, generator=g) * 3
    probes = torch.tensor([-80.0, -20.0, 0.0, 19.0, 19.999999, 20.0, 20.000001, 25.0, 80.0])
    a32[0, : len(probes)] = probes
    A = -torch.exp(torch.rand(H, generator=g) * 2)          # A = -exp(A_log), A_log ~ U(0, 2)
    dt_bias = torch.rand(H, generator=g) * 2 - 1            # U(-1, 1)
    dt_bias[: len(probes)] = 0
    out = {"A": A.numpy(), "dt_bias": dt_bias.numpy()}
    for name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        a = a32.to(dt)
        b = b32.to(dt)
        beta = torch.sigmoid(b).float()
        alpha = torch.exp(A * F.softplus(a.float() + dt_bias))
        out[f"a_{name}"] = a.float().numpy()
        out[f"b_{name}"] = b.float().numpy()
        out[f"alpha_{name}"] = alpha.numpy()
        out[f"beta_{name}"] = beta.numpy()
    np.savez_compressed(HERE / "gates_torch.npz", **out)


def e4m3_fixture():
    rng = np.random.default_rng(99)
    mags = np.exp(rng.uniform(np.log(1e-5), np.log(600.0), 20000))
    x = (mags * rng.choice([-1.0, 1.0], mags.size)).astype(np.float32)
    special = np.array([0.0, -0.0, 448.0, -448.0, 464.0, 464.00003, 472.0, 479.99997, 480.0,
                        2.0 ** -6, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -9, 2.5 * 2.0 ** -9,
                        3 * 2.0 ** -10, np.nan, -np.nan, np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([special, x])
    codes = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.savez_compressed(HERE / "e4m3fn_torch.npz", x=x, codes=codes)


def conv_fixture():
    rng = np.random.default_rng(5)
    B, C, K = 3, 64, 4
    window = rng.standard_normal((B, C, K)).astype(np.float32)
    x = rng.standard_normal((B, C)).astype(np.float32)
    w = (rng.standard_normal((C, K)) * 0.5).astype(np.float32)
    bias = (rng.standard_normal(C) * 0.1).astype(np.float32)
    out, win = conv_f64(window, x, w, bias)
    np.savez_compressed(HERE / "conv_f64.npz", window=window, x=x, weight=w, bias=bias,
                        out=out.astype(np.float32), window_out=win.astype(np.float32))


if __name__ == "__main__":
    decode_fixture()
    gates_fixture()
    e4m3_fixture()
    conv_fixture()
    print("fixtures written to", HERE)
