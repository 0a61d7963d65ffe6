"""Input builders and comparison helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

import oracle

DEV = "cuda"
KIND = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}

# Kernel-vs-oracle tolerance for fp32 arithmetic (the reference's own gate,
# tests/test_gdn_decode_kernel.py:36-37).
RTOL, ATOL = 2e-5, 2e-6
# The stated parity bar: outputs and fp32 final states within max-abs 2e-5 of
# the reference recurrence (fp32 math).
MAXABS = 2e-5


def gen(seed: int) -> torch.Generator:
    return torch.Generator(device=DEV).manual_seed(seed)


def decode_inputs(B, H=8, G=4, seed=0):
    g = gen(seed)
    return dict(
        q=torch.randn(B, G, 128, generator=g, device=DEV),
        k=torch.randn(B, G, 128, generator=g, device=DEV),
        v=torch.randn(B, H, 128, generator=g, device=DEV),
        alpha=torch.rand(B, H, generator=g, device=DEV) * 0.5 + 0.5,
        beta=torch.rand(B, H, generator=g, device=DEV),
    )


def prefill_inputs(B, T, H=8, G=4, seed=3):
    g = gen(seed)
    return dict(
        q=torch.randn(B, T, G, 128, generator=g, device=DEV),
        k=torch.randn(B, T, G, 128, generator=g, device=DEV),
        v=torch.randn(B, T, H, 128, generator=g, device=DEV),
        alpha=torch.rand(B, T, H, generator=g, device=DEV),
        beta=torch.rand(B, T, H, generator=g, device=DEV),
    )


def raw_gates(shape, H, dt, seed=7):
    """a_raw/b_raw of `shape` in the activation dtype plus A (= -exp(A_log)) and
    dt_bias, as the reference's tests draw them (test_gdn_raw_gates.py:72-83)."""
    g = gen(seed)
    a_raw = (torch.randn(*shape, generator=g, device=DEV) * 2).to(dt).contiguous()
    b_raw = (torch.randn(*shape, generator=g, device=DEV) * 2).to(dt).contiguous()
    A = -torch.exp(torch.randn(H, generator=g, device=DEV) * 0.5)
    dt_bias = torch.randn(H, generator=g, device=DEV) * 0.5
    return a_raw, b_raw, A.contiguous(), dt_bias.contiguous()


def torch_gates(a_raw, b_raw, A, dt_bias):
    """braid/model/gdn.py:299-300 exactly: sigmoid in the activation dtype then
    widened; alpha fp32 throughout. The in-kernel gates must equal this to the bit."""
    beta = torch.sigmoid(b_raw).float()
    alpha = torch.exp(A * F.softplus(a_raw.float() + dt_bias))
    return alpha.contiguous(), beta.contiguous()


def pool(S, H=8, dtype=torch.float32, seed=11, scale=0.1):
    p = torch.randn(S, H, 128, 128, generator=gen(seed), device=DEV) * scale
    return p.to(dtype).contiguous()


def to_np_pool(p: torch.Tensor) -> np.ndarray:
    """A device pool as the oracle's storage array."""
    if p.dtype == torch.bfloat16:
        return p.view(torch.uint16).cpu().numpy().copy()
    return p.cpu().numpy().copy()


def act_np(t: torch.Tensor) -> np.ndarray:
    """Activation tensor for the oracle: fp32 values, or bf16 bit patterns."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.uint16).cpu().numpy()
    return t.float().cpu().numpy()


def ulp16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in units in the last place between two arrays of 16-bit floats
    (fp16 arrays, or bf16 bit patterns as uint16)."""
    def ordered(x):
        u = np.asarray(x).view(np.uint16).astype(np.int64)
        return np.where(u & 0x8000, 0x8000 - u, u)
    return np.abs(ordered(a) - ordered(b))


def assert_parity(got, ref, what: str = "", maxabs: float = MAXABS, rel: bool = True):
    """Kernel output against the oracle: max-abs error <= `maxabs` (printed),
    and with `rel` also the reference's relative gate (RTOL, ATOL)."""
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    worst = float(np.nanmax(err)) if err.size else 0.0
    print(f"  parity {what or 'output'}: max-abs {worst:.3e} (bar {maxabs:.0e}) over "
          f"{err.size} values", flush=True)
    assert not np.isnan(err).any(), f"{what}: NaN where the oracle has a number"
    assert worst <= maxabs, f"{what}: max-abs error {worst:.3e} exceeds {maxabs:.0e}"
    if rel:
        np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL, err_msg=what)


def assert_pool_close(kern_pool: torch.Tensor, ref: np.ndarray, rows, what=""):
    """fp32 pools within the fp32 tolerance; 16-bit pools within one ulp of
    the element, plus 2^-20 of the slab's rms for elements that cancellation
    left near zero: the kernel and the oracle sum kv in different fp32
    orders, which moves a result by ~1e-7 of the state's scale, and that is
    several ulps of an element a thousand times smaller than the rest (still
    ~4000x below one ulp at the state's scale)."""
    got = to_np_pool(kern_pool)[rows]
    exp = ref[rows]
    if kern_pool.dtype == torch.float32:
        assert_parity(got, exp, what or "fp32 state")
        return
    kind = "f16" if kern_pool.dtype == torch.float16 else "bf16"
    g = oracle.widen(got, kind).astype(np.float64)
    r = oracle.widen(exp, kind).astype(np.float64)
    rms = float(np.sqrt(np.mean(r * r)))
    bound = ulp_of(r, kind).astype(np.float64) + 2.0 ** -20 * rms
    err = np.abs(g - r)
    d = ulp16(got, exp)
    print(f"  {what or 'narrow state'}: {int((d > 1).sum())} of {d.size} elements beyond 1 ulp "
          f"(max {int(d.max())}), worst {float((err / bound).max()):.2f}x the bound", flush=True)
    assert (err <= bound).all(), (f"{what}: {int((err > bound).sum())} elements beyond one ulp "
                                  f"+ 2^-20 rms")


def ulp_of(x: np.ndarray, kind: str) -> np.ndarray:
    """Spacing of the storage type at |x| (x given as float32 values)."""
    x = np.abs(np.asarray(x, np.float32))
    if kind == "f16":
        return np.spacing(x.astype(np.float16)).astype(np.float32)
    if kind == "bf16":
        return np.maximum(np.spacing(x) * 65536.0, np.float32(2.0 ** -133))
    return np.spacing(x)


def assert_free_running_close(got_bits: np.ndarray, ref_bits: np.ndarray, kind: str, ulps=2):
    """Multi-token comparison of a narrow pool against the oracle. Each token
    may round the two sides one ulp apart and later tokens carry that forward
    (non-expansively), so the bound is a few ulps of the element OR of the
    state's typical magnitude (near-zero elements have tiny ulps)."""
    g = oracle.widen(got_bits, kind)
    r = oracle.widen(ref_bits, kind)
    rms = np.float32(np.sqrt(np.mean(r.astype(np.float64) ** 2)))
    bound = ulps * (ulp_of(r, kind) + ulp_of(rms, kind))
    err = np.abs(g - r)
    bad = err > bound
    assert not bad.any(), (f"{int(bad.sum())} elements beyond {ulps} ulp; worst "
                           f"{float((err / bound).max()):.2f}x the bound")
