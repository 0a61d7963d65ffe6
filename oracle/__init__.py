"""CPU oracle for the GDN mixer hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or, for
the baseline, as the thing timed on the host). The product path —
``braid_amd`` and ``libbraid_gdn.so`` — never imports, links or calls it.

The arithmetic lives in ``gdn_oracle.c`` (scalar fp32, no contraction, libm
transcendentals); this module is the numpy-facing wrapper that gathers and
scatters slot-indexed pools and emulates the pool storage types:

* ``"f32"`` pools are float32 arrays;
* ``"f16"`` pools are float16 arrays (numpy's float32->float16 cast rounds to
  nearest even, as the kernel's conversion does);
* ``"bf16"`` pools are uint16 arrays of bfloat16 bit patterns (round to
  nearest even, NaN -> 0x7FC0).

Reference lines each function restates are cited in ``gdn_oracle.c``; the
wrappers add only the pool bookkeeping of braid/kernels/csrc/gdn_decode.cu
(slot-indexed rows, state widened on load and narrowed once per token on
store) and braid/kernels/csrc/conv1d_decode.cu:21-27 (window layout).

Pinning (what checks this oracle, in tests/test_oracle.py): brute-force
float64 Python loops on tiny shapes, a float64 numpy closed form at full
shape, the reference's own invariants (beta=0 is pure decay, rows
independent, grouped head->group map, pad identity, chunk split), the
softplus threshold probes, torch's CPU spelling of the gates, of the
gated RMSNorm readout and of the fp8 cast, and exhaustive e4m3fn round-trips.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i32, _i64 = ctypes.c_int, ctypes.c_int64

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from oracle.build import build
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_gdn_decode.argtypes = [_f32p, _i32, _i32, _i32, _i32, _i32, _f32p, _i64,
                                        _f32p, _i64, _f32p, _i64, _f32p, _f32p, _f32p, _f32p]
        L.oracle_gdn_decode.restype = None
        L.oracle_gdn_gates.argtypes = [_f32p, _f32p, _i32, _i32, _i32, _f32p, _f32p, _i32,
                                       ctypes.c_void_p, _f32p, _f32p]
        L.oracle_gdn_gates.restype = None
        L.oracle_conv1d_decode.argtypes = [_f32p, _i32, _i32, _i32, _f32p, _f32p,
                                           ctypes.c_void_p, _f32p]
        L.oracle_conv1d_decode.restype = None
        L.oracle_quantize_act.argtypes = [_f32p, _i64, _u8p, ctypes.POINTER(ctypes.c_float)]
        L.oracle_quantize_act.restype = None
        L.oracle_e4m3fn.argtypes = [ctypes.c_float]
        L.oracle_e4m3fn.restype = ctypes.c_uint8
        L.oracle_bf16_round.argtypes = [ctypes.c_float]
        L.oracle_bf16_round.restype = ctypes.c_float
        _lib = L
    return _lib


# ---- storage emulation ----------------------------------------------------

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    out = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    out[nan] = 0x7FC0
    return out


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def widen(a: np.ndarray, kind: str) -> np.ndarray:
    if kind == "f32":
        return np.array(a, dtype=np.float32)
    if kind == "f16":
        return np.asarray(a, dtype=np.float16).astype(np.float32)
    if kind == "bf16":
        return bf16_value(a)
    raise ValueError(kind)


def narrow(a: np.ndarray, kind: str) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    if kind == "f32":
        return a.copy()
    if kind == "f16":
        with np.errstate(over="ignore"):
            return a.astype(np.float16)
    if kind == "bf16":
        return bf16_bits(a)
    raise ValueError(kind)


def _c(a, dtype=np.float32) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- GDN ---------------------------------------------------------------------

def gdn_decode_rows(state: np.ndarray, q, k, v, alpha, beta) -> np.ndarray:
    """One token on fp32 states [B, H, SS, HD] (updated in place); raw q, k
    [B, G, SS] (normalised inside); v [B, H, HD]; alpha, beta [B, H].
    Returns y [B, H, HD]."""
    assert state.dtype == np.float32 and state.flags.c_contiguous
    B, H, SS, HD = state.shape
    q, k, v = _c(q), _c(k), _c(v)
    G = q.shape[1]
    y = np.empty((B, H, HD), dtype=np.float32)
    scratch = np.empty(2 * SS + 2 * HD, dtype=np.float32)
    lib().oracle_gdn_decode(state, B, H, G, SS, HD, q, G * SS, k, G * SS, v, H * HD,
                            _c(alpha), _c(beta), y, scratch)
    return y


def gdn_decode(pool: np.ndarray, slot_idx, q, k, v, alpha, beta, kind: str) -> np.ndarray:
    """Decode step over a slot-indexed pool [S, H, SS, HD] stored as `kind`
    (updated in place at slot_idx rows). Returns y [B, H, HD]."""
    idx = np.asarray(slot_idx, dtype=np.int64)
    st = np.ascontiguousarray(widen(pool[idx], kind))
    y = gdn_decode_rows(st, q, k, v, alpha, beta)
    pool[idx] = narrow(st, kind)
    return y


def gdn_prefill(pool: np.ndarray, slot_idx, q, k, v, alpha, beta, kind: str) -> np.ndarray:
    """T tokens: q, k [B, T, G, SS], v [B, T, H, HD], alpha/beta [B, T, H].
    The state is narrowed to the pool type after every token, the contract
    that makes the chunk scan equal to T decode steps. Returns y [B,T,H,HD]."""
    idx = np.asarray(slot_idx, dtype=np.int64)
    B, T = q.shape[:2]
    H, HD = v.shape[2], v.shape[3]
    y = np.empty((B, T, H, HD), dtype=np.float32)
    st = np.ascontiguousarray(widen(pool[idx], kind))
    for t in range(T):
        y[:, t] = gdn_decode_rows(st, q[:, t], k[:, t], v[:, t], alpha[:, t], beta[:, t])
        st = np.ascontiguousarray(widen(narrow(st, kind), kind))
    pool[idx] = narrow(st, kind)
    return y


def gdn_gates(a_raw, b_raw, A, dt_bias, act: str = "f32",
              seq_lens: Optional[np.ndarray] = None):
    """alpha, beta for raw projections [B, H] or [B, T, H].

    `act` is the activation dtype: "f32" (a_raw/b_raw float32) or "bf16"
    (uint16 bit patterns; beta's sigmoid is rounded through bf16).
    """
    a_raw = np.asarray(a_raw)
    shape = a_raw.shape
    B, H = shape[0], shape[-1]
    T = 1 if len(shape) == 2 else shape[1]
    af = widen(a_raw, act).reshape(-1)
    bf = widen(np.asarray(b_raw), act).reshape(-1)
    alpha = np.empty(af.shape, dtype=np.float32)
    beta = np.empty(af.shape, dtype=np.float32)
    sl = None
    if seq_lens is not None:
        sl_arr = _c(seq_lens, np.int32)
        sl = sl_arr.ctypes.data_as(ctypes.c_void_p)
    lib().oracle_gdn_gates(_c(af), _c(bf), B, T, H, _c(A), _c(dt_bias),
                           1 if act == "bf16" else 0, sl, alpha, beta)
    return alpha.reshape(shape), beta.reshape(shape)


# ---- conv --------------------------------------------------------------------

def conv1d_decode(conv_pool: np.ndarray, slot_idx, x, weight, bias) -> np.ndarray:
    """conv_pool [S, C, K] fp32 updated in place at slot_idx rows; x [B, C]
    fp32; weight [C, K]; bias [C] or None. Returns out [B, C]."""
    idx = np.asarray(slot_idx, dtype=np.int64)
    st = np.ascontiguousarray(conv_pool[idx], dtype=np.float32)
    B, C, K = st.shape
    out = np.empty((B, C), dtype=np.float32)
    bias_arr = None if bias is None else _c(bias)
    bp = None if bias_arr is None else bias_arr.ctypes.data_as(ctypes.c_void_p)
    lib().oracle_conv1d_decode(st, B, C, K, _c(x), _c(weight), bp, out)
    conv_pool[idx] = st
    return out


def conv1d_prefill(conv_pool: np.ndarray, slot_idx, x, weight, bias, seq_lens=None):
    """T tokens of the decode step per row: x [B, T, C] fp32; row b runs tokens
    0..min(seq_lens[b], T)-1 (all T when seq_lens is None); pad outputs are 0
    and leave the window alone. Returns out [B, T, C]."""
    x = _c(x)
    B, T, C = x.shape
    out = np.zeros((B, T, C), dtype=np.float32)
    idx = np.asarray(slot_idx, dtype=np.int64)
    for b in range(B):
        n = T if seq_lens is None else int(min(max(int(seq_lens[b]), 0), T))
        for t in range(n):
            out[b, t] = conv1d_decode(conv_pool, idx[b:b + 1], x[b:b + 1, t], weight, bias)[0]
    return out


# ---- gated RMSNorm readout ------------------------------------------------------

def gated_rmsnorm(y: np.ndarray, z: np.ndarray, gamma: np.ndarray, eps: float,
                  act: str) -> np.ndarray:
    """Readout of the scan, restating braid/model/gdn.py:373-387 (`_readout`:
    ``y.to(dtype)``) and braid/model/norm.py:48-71 (`rms_norm_gated`):

        c    = round_act(y)
        xf   = c * rsqrt(mean(c^2) + eps)         over the last axis (HD)
        h    = gamma * round_act(xf)               fp32 (gamma is fp32)
        core = round_act(h * (zf / (1 + exp(-zf))))

    y: fp32 values [..., HD]; z: the gate in act storage (uint16 bf16 bits,
    float16, or float32); gamma [HD] fp32. Returns core in act storage. The
    mean of squares is summed in float64 and rounded once to fp32, and the
    reciprocal square root of the fp32 sum ``mean + eps`` is correctly rounded
    (torch's fp32 reduction and rsqrt differ from these only in rounding).
    Every other step is one fp32 operation, rounded as torch does.
    """
    c = widen(narrow(y, act), act)
    ms = np.square(c.astype(np.float64)).mean(axis=-1, keepdims=True)
    t = (ms.astype(np.float32) + np.float32(eps)).astype(np.float32)
    r = (1.0 / np.sqrt(t.astype(np.float64))).astype(np.float32)
    xf = (c * r).astype(np.float32)
    xb = widen(narrow(xf, act), act)
    h = (np.asarray(gamma, dtype=np.float32) * xb).astype(np.float32)
    zf = widen(z, act)
    with np.errstate(over="ignore"):
        s = (zf / (np.float32(1.0) + np.exp(-zf))).astype(np.float32)
    o = (h * s).astype(np.float32)
    return narrow(o, act)


# ---- FP8 ---------------------------------------------------------------------

def quantize_act(x: np.ndarray):
    """x (float32 values of the activation) -> (codes uint8 of x's shape,
    scale float32)."""
    xf = _c(x).reshape(-1)
    q = np.empty(xf.shape, dtype=np.uint8)
    sc = ctypes.c_float()
    lib().oracle_quantize_act(xf, xf.size, q, ctypes.byref(sc))
    return q.reshape(np.shape(x)), np.float32(sc.value)


def e4m3fn(x) -> np.ndarray:
    """Elementwise float32 -> e4m3fn code (uint8)."""
    f = lib().oracle_e4m3fn
    xs = _c(x).reshape(-1)
    return np.array([f(float(v)) for v in xs], dtype=np.uint8).reshape(np.shape(x))


def bf16_round(x: float) -> float:
    return lib().oracle_bf16_round(x)
