"""``load_gdn()``: the GDN hot-path entry points over the C ABI.

Drop-in for ``braid.kernels.loader.load_gdn`` (braid/kernels/loader.py:10-44),
which JIT-built a pybind11 module exposing ``gdn_decode``, ``gdn_prefill``,
``gdn_decode_raw``, ``gdn_prefill_raw``, ``conv1d_decode`` and ``quantize_act``
(braid/kernels/csrc/bindings.cpp:25-34). Here the kernels live in the
prebuilt gfx950 library ``braid_amd/libbraid_gdn.so`` (C ABI declared in
``include/braid_gdn.h``) and this module is the thin torch-facing layer:

* the same call signatures, argument meaning and in-place semantics;
* the same argument checks, raising ``RuntimeError`` with the message
  fragments the reference's tests match ("rows overlap", "out of range",
  "duplicate ... distinct", "only SS=HD=128", ...);
* work is enqueued on torch's current stream of the pool's device, with no
  implicit synchronisation except the eager slot validation the library
  performs (skipped while the stream is capturing a graph);
* ``quantize_act`` allocates its outputs (and the small partial-max
  workspace) in torch, as the reference's did.

Beyond the reference's six, the object fronts the rows this build adds on
either side of the scan: ``conv1d_prefill`` (the prefill conv the reference
ran in torch), ``gdn_conv_decode_raw`` (conv1d_decode + gdn_decode_raw in one
launch), ``gated_rmsnorm`` (the readout and the out_proj input quantization)
and ``fp8_matmul`` (the FP8 GEMM, hipBLASLt).

There is no CPU or torch fallback: if the library is missing or a tensor is
not on the GPU, the call raises.
"""
from __future__ import annotations

import contextlib
import ctypes
from functools import lru_cache
from pathlib import Path
from typing import Optional, Sequence

import torch

LIB_PATH = Path(__file__).resolve().parent.parent / "libbraid_gdn.so"

BRAID_F32, BRAID_F16, BRAID_BF16 = 0, 1, 2
_POOL_DTYPES = {torch.float32: BRAID_F32, torch.float16: BRAID_F16,
                torch.bfloat16: BRAID_BF16}
_ACT_DTYPES = {torch.float32: BRAID_F32, torch.bfloat16: BRAID_BF16}
_QUANT_DTYPES = {torch.float32: BRAID_F32, torch.float16: BRAID_F16,
                 torch.bfloat16: BRAID_BF16}

_vp, _i32, _i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64

# Argument lists of the exported entry points, in include/braid_gdn.h order.
SIGNATURES = {
    "braid_abi_version": ([], _i32),
    "braid_last_error": ([], ctypes.c_char_p),
    "braid_set_launch_override": ([_i32, _i32], _i32),
    "braid_get_launch_override": ([_i32], _i32),
    "braid_prefill_plan": ([_vp, _i32, _i32, _i32, _i32], _i32),
    "braid_gdn_decode": ([_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32,
                          _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp], _i32),
    "braid_gdn_decode_raw": ([_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32,
                              _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i32,
                              _vp, _vp, _vp, _vp], _i32),
    "braid_gdn_prefill": ([_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _i32,
                           _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "braid_gdn_prefill_raw": ([_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _i32,
                               _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp,
                               _vp], _i32),
    "braid_gdn_prefill_raw_plan": ([_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _i32,
                                    _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp,
                                    _i32, _vp], _i32),
    "braid_gdn_conv_decode_raw": ([_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _vp,
                                   _i32, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp,
                                   _vp], _i32),
    "braid_conv1d_decode": ([_vp, _i64, _i32, _i32, _vp, _i32, _vp, _i32, _vp, _vp,
                             _vp, _vp], _i32),
    "braid_conv1d_prefill": ([_vp, _i64, _i32, _i32, _vp, _i32, _i32, _vp, _i32, _vp, _vp,
                              _vp, _vp, _vp], _i32),
    "braid_quantize_act_workspace": ([_i64], _i32),
    "braid_quantize_act": ([_vp, _i32, _i64, _vp, _vp, _vp, _vp], _i32),
    "braid_quantize_act_noalloc": ([_vp, _i32, _i64, _vp, _vp, _vp], _i32),
    "braid_gated_rmsnorm_workspace": ([_i64], _i32),
    "braid_fp8_gemm_workspace": ([], ctypes.c_size_t),
    "braid_fp8_gemm": ([_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp, ctypes.c_size_t,
                        _vp], _i32),
    "braid_gated_rmsnorm_quant": ([_vp, _i32, _vp, _i32, _vp, ctypes.c_float, _i64, _i32, _vp,
                                   _vp, _vp, _vp, _vp], _i32),
}


def open_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    """dlopen the kernel library and declare every entry point's prototype.

    torch is imported first on purpose: the library links ``libamdhip64.so.7``
    and the dynamic linker then binds it to the HIP runtime torch already
    loaded, so torch's streams and device pointers are valid in it.
    """
    if not path.exists():
        raise RuntimeError(
            f"{path.name} is not built at {path}; run `python -m braid_amd.build` "
            "(the GDN kernels have no fallback)")
    lib = ctypes.CDLL(str(path))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _row_stride_3d(t: torch.Tensor, name: str, require_cuda: bool = True) -> int:
    """Batch stride of a [B, X, Y] fp32 operand whose last two dims are dense
    (gdn_decode.cu:303-311): only the batch stride may differ, and rows may
    not overlap."""
    # The messages are built only on failure: formatting them on every call
    # cost more than the checks.
    if not ((t.is_cuda or not require_cuda) and t.dtype == torch.float32):
        raise RuntimeError(f"{name} must be cuda fp32")
    if t.dim() != 3:
        raise RuntimeError(f"{name} must be 3-d")
    s0, s1, s2 = t.stride()
    n0, n1, n2 = t.shape
    if not (s2 == 1 and s1 == n2):
        raise RuntimeError(f"{name} must be dense in its last two dims (only the batch stride "
                           f"may differ; got strides {(s0, s1, s2)})")
    if not (n0 <= 1 or s0 >= n1 * n2):
        raise RuntimeError(f"{name} rows overlap")
    return max(s0, n1 * n2)


def _check_pool(pool: torch.Tensor, slot_idx: torch.Tensor) -> int:
    _check(pool.is_cuda, "pool must be cuda")
    _check(pool.dtype in _POOL_DTYPES, "state pool must be fp32, fp16 or bf16")
    _check(slot_idx.dtype == torch.int32, "slot_idx must be int32")
    _check(slot_idx.is_cuda and slot_idx.is_contiguous(), "slot_idx must be contiguous cuda")
    _check(pool.is_contiguous(), "pool must be contiguous")
    _check(pool.dim() == 4, "pool shape must be [S_max, H, SS, HD]")
    return _POOL_DTYPES[pool.dtype]


def _check_dense_f32(ts, msg: str) -> None:
    for t in ts:
        _check(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous(), msg)


def _check_raw(a_raw, b_raw, A, dt_bias) -> int:
    _check(a_raw.dtype in _ACT_DTYPES,
           "a_raw/b_raw must be fp32 or bf16 (the activation dtypes braid runs)")
    _check(b_raw.dtype == a_raw.dtype, "a_raw and b_raw must share a dtype")
    for t in (a_raw, b_raw):
        _check(t.is_cuda and t.is_contiguous(), "a_raw/b_raw must be contiguous cuda")
    _check_dense_f32((A, dt_bias), "A/dt_bias must be contiguous cuda fp32")
    return _ACT_DTYPES[a_raw.dtype]


class GDNKernels:
    """The loaded module: one method per reference entry point."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib
        self.abi_version = lib.braid_abi_version()
        self._workspaces: dict = {}

    # -- plumbing -------------------------------------------------------------

    def _call(self, fn_name: str, device: torch.device, *args) -> None:
        # The library launches on the current HIP device; switch to the
        # operands' device only when it is another one (the switch costs
        # about 3 us a call).
        if device.index is None or device.index == torch.cuda.current_device():
            rc = getattr(self._lib, fn_name)(*args, torch.cuda.current_stream().cuda_stream)
        else:
            with torch.cuda.device(device):
                stream = torch.cuda.current_stream(device).cuda_stream
                rc = getattr(self._lib, fn_name)(*args, stream)
        if rc != 0:
            raise RuntimeError(self._lib.braid_last_error().decode())

    # -- launch knobs (measurement / tests) ------------------------------------

    KNOBS = {"decode_xcd_remap": 0, "decode_wgs_per_cu": 1, "prefill_layout": 2,
             "decode_parts": 3, "prefill_plan": 4, "fp8_gemm": 5}

    @contextlib.contextmanager
    def launch_override(self, **knobs):
        """Force launch-shape choices for the calls inside the block (None:
        the library's own choice), restoring the previous values after. Only
        the time changes; every shape gives the same bits, except fp8_gemm,
        which picks between two GEMMs that sum in different orders."""
        prev = {}
        try:
            for name, val in knobs.items():
                knob = self.KNOBS[name]
                prev[knob] = self._lib.braid_get_launch_override(knob)
                rc = self._lib.braid_set_launch_override(knob, -1 if val is None else int(val))
                _check(rc == 0, self._lib.braid_last_error().decode())
            yield
        finally:
            for knob, val in prev.items():
                self._lib.braid_set_launch_override(knob, val)

    # -- GDN scans ------------------------------------------------------------

    def gdn_decode(self, pool, slot_idx, q, k, v, alpha, beta, y) -> None:
        """One token for B rows; pool updated in place at slot_idx rows
        (gdn_decode.cu:313-360)."""
        pdt = _check_pool(pool, slot_idx)
        _check_dense_f32((alpha, beta, y), "alpha/beta/y must be contiguous cuda fp32")
        q_row, k_row, v_row = (_row_stride_3d(q, "q"), _row_stride_3d(k, "k"),
                               _row_stride_3d(v, "v"))
        B, G, SS = q.shape
        H, HD = v.size(1), v.size(2)
        self._check_decode_shapes(pool, slot_idx, q, k, v, y, B, G, SS, H, HD)
        _check(alpha.numel() == B * H and beta.numel() == B * H, "alpha/beta must be [B, H]")
        self._call("braid_gdn_decode", pool.device, _ptr(pool), pdt, pool.size(0), H, G, SS,
                   HD, _ptr(slot_idx), B, _ptr(q), q_row, _ptr(k), k_row, _ptr(v), v_row,
                   _ptr(alpha), _ptr(beta), _ptr(y))

    def gdn_decode_raw(self, pool, slot_idx, q, k, v, a_raw, b_raw, A, dt_bias, y) -> None:
        """Decode with alpha/beta computed in-kernel from the raw projections
        (gdn_decode.cu:367-441)."""
        pdt = _check_pool(pool, slot_idx)
        _check(y.is_cuda and y.dtype == torch.float32 and y.is_contiguous(),
               "y must be contiguous cuda fp32")
        q_row, k_row, v_row = (_row_stride_3d(q, "q"), _row_stride_3d(k, "k"),
                               _row_stride_3d(v, "v"))
        adt = _check_raw(a_raw, b_raw, A, dt_bias)
        B, G, SS = q.shape
        H, HD = v.size(1), v.size(2)
        self._check_decode_shapes(pool, slot_idx, q, k, v, y, B, G, SS, H, HD)
        _check(a_raw.dim() >= 1 and a_raw.size(0) == B and a_raw.numel() == B * H,
               "a_raw must be [B, H]")
        _check(b_raw.shape == a_raw.shape, "b_raw must match a_raw")
        _check(A.numel() == H and dt_bias.numel() == H, "A and dt_bias must be [H]")
        self._call("braid_gdn_decode_raw", pool.device, _ptr(pool), pdt, pool.size(0), H, G,
                   SS, HD, _ptr(slot_idx), B, _ptr(q), q_row, _ptr(k), k_row, _ptr(v), v_row,
                   _ptr(a_raw), _ptr(b_raw), adt, _ptr(A), _ptr(dt_bias), _ptr(y))

    def gdn_conv_decode_raw(self, pool, conv_pool, slot_idx, x, weight, bias, a_raw, b_raw,
                            A, dt_bias, y, n_groups: int) -> None:
        """conv1d_decode then gdn_decode_raw on the conv output's q/k/v views,
        fused in one launch with the same bits (gdn.py:131-160). x [B, C] is
        the pre-conv projection (fp32 or bf16), C = 2 * n_groups * 128 + H * 128;
        the conv output is not materialised."""
        pdt = _check_pool(pool, slot_idx)
        _check(conv_pool.is_cuda and conv_pool.dtype == torch.float32
               and conv_pool.is_contiguous() and conv_pool.dim() == 3,
               "conv_pool must be contiguous cuda fp32 [S_max, C, K]")
        _check(y.is_cuda and y.dtype == torch.float32 and y.is_contiguous(),
               "y must be contiguous cuda fp32")
        adt = _check_raw(a_raw, b_raw, A, dt_bias)
        n_slots, H, SS, HD = pool.shape
        G = int(n_groups)
        _check(G > 0 and H % G == 0, "n_heads must be divisible by n_groups")
        C, K = conv_pool.size(1), conv_pool.size(2)
        _check(C == 2 * G * SS + H * HD, "conv_pool channels must be 2*G*SS + H*HD")
        _check(conv_pool.size(0) == n_slots, "conv_pool and pool must hold the same slots")
        _check(x.dim() == 2 and x.size(1) == C, "x must be [B, C]")
        B = x.size(0)
        _check(x.dtype in _ACT_DTYPES, "x must be fp32 or bf16 (the activation dtypes braid runs)")
        _check(x.is_cuda and x.is_contiguous(), "x must be contiguous")
        _check(tuple(weight.shape) == (C, K), "weight must be [C, K]")
        _check_dense_f32((weight,), "weight must be contiguous cuda fp32")
        bias_p = None
        if bias is not None and bias.numel() > 0:
            _check_dense_f32((bias,), "bias must be contiguous cuda fp32")
            _check(bias.numel() == C, "bias must be [C]")
            bias_p = _ptr(bias)
        _check(slot_idx.numel() == B, "slot_idx must have one entry per batch row")
        _check(tuple(y.shape) == (B, H, HD), "y shape must be [B, H, HD]")
        _check(a_raw.numel() == B * H and b_raw.shape == a_raw.shape, "a_raw/b_raw must be [B, H]")
        _check(A.numel() == H and dt_bias.numel() == H, "A and dt_bias must be [H]")
        self._call("braid_gdn_conv_decode_raw", pool.device, _ptr(pool), pdt, n_slots, H, G, SS,
                   HD, _ptr(conv_pool), K, _ptr(slot_idx), B, _ptr(x), _ACT_DTYPES[x.dtype],
                   _ptr(weight), bias_p, _ptr(a_raw), _ptr(b_raw), adt, _ptr(A), _ptr(dt_bias),
                   _ptr(y))

    @staticmethod
    def _check_decode_shapes(pool, slot_idx, q, k, v, y, B, G, SS, H, HD) -> None:
        _check(SS == 128 and HD == 128, "only SS=HD=128 is instantiated")
        _check(H % G == 0, "n_heads must be divisible by n_groups")
        _check(k.shape == q.shape, "k must match q")
        _check(v.size(0) == B, "v must match q in B")
        _check(slot_idx.numel() == B, "slot_idx must have one entry per batch row")
        _check(tuple(pool.shape[1:]) == (H, SS, HD), "pool shape must be [S_max, H, SS, HD]")
        _check(tuple(y.shape) == (B, H, HD), "y shape must be [B, H, HD]")

    def gdn_prefill(self, pool, slot_idx, q, k, v, alpha, beta, y) -> None:
        """T tokens per launch, state on chip between them
        (gdn_decode.cu:553-603). Caller pads with alpha=1, beta=0."""
        pdt = _check_pool(pool, slot_idx)
        _check_dense_f32((q, k, v, alpha, beta, y), "all operands must be contiguous cuda fp32")
        B, T, G, SS, H, HD = self._check_prefill_shapes(pool, slot_idx, q, k, v, y)
        _check(tuple(alpha.shape) == (B, T, H), "alpha must be [B, T, H]")
        _check(beta.shape == alpha.shape, "beta must match alpha")
        self._call("braid_gdn_prefill", pool.device, _ptr(pool), pdt, pool.size(0), H, G, SS,
                   HD, _ptr(slot_idx), B, T, _ptr(q), _ptr(k), _ptr(v), _ptr(alpha),
                   _ptr(beta), _ptr(y))

    def gdn_prefill_raw(self, pool, slot_idx, q, k, v, a_raw, b_raw, A, dt_bias, y,
                        seq_lens: Optional[torch.Tensor] = None,
                        plan_lens: Optional[Sequence[int]] = None) -> None:
        """Chunk scan with in-kernel gates and ragged seq_lens
        (gdn_decode.cu:611-699). seq_lens=None means every column is live.

        ``plan_lens``: the row lengths, on the host, to plan a ragged launch
        from when the call cannot read ``seq_lens`` itself, that is under graph
        capture (an eager call plans from ``seq_lens`` and ignores it). A
        graph captured with them keeps that plan for every replay; the results
        are the same bits for whatever lengths a replay holds, only the time
        depends on the plan. Not in the reference, whose prefill is eager."""
        pdt = _check_pool(pool, slot_idx)
        _check_dense_f32((q, k, v, y), "q/k/v/y must be contiguous cuda fp32")
        adt = _check_raw(a_raw, b_raw, A, dt_bias)
        B, T, G, SS, H, HD = self._check_prefill_shapes(pool, slot_idx, q, k, v, y)
        _check(a_raw.dim() >= 2 and a_raw.size(0) == B and a_raw.size(1) == T
               and a_raw.numel() == B * T * H, "a_raw must be [B, T, H]")
        _check(b_raw.shape == a_raw.shape, "b_raw must match a_raw")
        _check(A.numel() == H and dt_bias.numel() == H, "A and dt_bias must be [H]")
        if seq_lens is not None:
            _check(seq_lens.is_cuda and seq_lens.dtype == torch.int32
                   and seq_lens.is_contiguous(), "seq_lens must be contiguous cuda int32")
            _check(seq_lens.numel() == B, "seq_lens must have one entry per batch row")
        if plan_lens is None:
            self._call("braid_gdn_prefill_raw", pool.device, _ptr(pool), pdt, pool.size(0), H,
                       G, SS, HD, _ptr(slot_idx), B, T, _ptr(q), _ptr(k), _ptr(v), _ptr(a_raw),
                       _ptr(b_raw), adt, _ptr(A), _ptr(dt_bias), _ptr(y), _ptr(seq_lens))
            return
        _check(seq_lens is not None, "plan_lens plans a ragged batch: seq_lens is required")
        _check(len(plan_lens) == B, "plan_lens must have one entry per batch row")
        plan = self.prefill_plan(plan_lens, T, H, pool.device)
        self._call("braid_gdn_prefill_raw_plan", pool.device, _ptr(pool), pdt, pool.size(0), H,
                   G, SS, HD, _ptr(slot_idx), B, T, _ptr(q), _ptr(k), _ptr(v), _ptr(a_raw),
                   _ptr(b_raw), adt, _ptr(A), _ptr(dt_bias), _ptr(y), _ptr(seq_lens), plan)

    def prefill_plan(self, lens: Sequence[int], T: int, H: int, device=None) -> int:
        """The plan (n8 * 2^20 + n4 * 2^10 + n2) an eager ragged prefill of
        these host lengths runs on ``device`` (braid_prefill_plan)."""
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        arr = (ctypes.c_int32 * len(lens))(*[int(x) for x in lens])
        plan = self._lib.braid_prefill_plan(ctypes.cast(arr, ctypes.c_void_p), len(lens), T, H,
                                            cus)
        _check(plan >= 0, self._lib.braid_last_error().decode())
        return plan

    @staticmethod
    def _check_prefill_shapes(pool, slot_idx, q, k, v, y):
        _check(q.dim() == 4 and v.dim() == 4, "q/k must be [B, T, G, SS], v [B, T, H, HD]")
        B, T, G, SS = q.shape
        H, HD = v.size(2), v.size(3)
        _check(SS == 128 and HD == 128, "only SS=HD=128 is instantiated")
        _check(H % G == 0, "n_heads must be divisible by n_groups")
        _check(slot_idx.numel() == B, "slot_idx must have one entry per batch row")
        _check(k.shape == q.shape, "k must match q")
        _check(v.size(0) == B and v.size(1) == T, "v must match q in [B, T]")
        _check(tuple(pool.shape[1:]) == (H, SS, HD), "pool shape must be [S_max, H, SS, HD]")
        _check(tuple(y.shape) == (B, T, H, HD), "y shape must be [B, T, H, HD]")
        return B, T, G, SS, H, HD

    # -- conv -----------------------------------------------------------------

    def conv1d_decode(self, conv_pool, slot_idx, x, weight, bias, out) -> None:
        """Slotted causal conv1d decode step + SiLU (conv1d_decode.cu:91-149).
        `bias` may be None or empty."""
        _check(conv_pool.is_cuda and conv_pool.dtype == torch.float32,
               "conv_pool must be cuda fp32")
        _check(conv_pool.is_contiguous(), "conv_pool must be contiguous")
        _check(slot_idx.dtype == torch.int32, "slot_idx must be int32")
        _check(slot_idx.is_cuda and slot_idx.is_contiguous(), "slot_idx must be contiguous cuda")
        _check(conv_pool.dim() == 3, "conv_pool must be [S_max, C, K]")
        n_slots, C, K = conv_pool.shape
        B = x.size(0)
        _check(K <= 8, "conv_kernel > 8 is not instantiated")
        _check(x.dim() == 2 and x.size(1) == C and tuple(out.shape) == (B, C),
               "x/out must be [B, C]")
        _check(tuple(weight.shape) == (C, K), "weight must be [C, K]")
        _check_dense_f32((weight,), "weight must be contiguous cuda fp32")
        _check(slot_idx.numel() == B, "slot_idx must have one entry per batch row")
        _check(x.dtype in _ACT_DTYPES,
               "x must be fp32 or bf16 (the activation dtypes braid runs)")
        _check(x.is_cuda and x.is_contiguous(), "x must be contiguous")
        _check(out.is_cuda and out.dtype == torch.float32 and out.is_contiguous(),
               "out must be contiguous fp32")
        bias_p = None
        if bias is not None and bias.numel() > 0:
            _check_dense_f32((bias,), "bias must be contiguous cuda fp32")
            _check(bias.numel() == C, "bias must be [C]")
            bias_p = _ptr(bias)
        self._call("braid_conv1d_decode", conv_pool.device, _ptr(conv_pool), n_slots, C, K,
                   _ptr(slot_idx), B, _ptr(x), _ACT_DTYPES[x.dtype], _ptr(weight), bias_p,
                   _ptr(out))

    def conv1d_prefill(self, conv_pool, slot_idx, x, weight, bias, out,
                       seq_lens: Optional[torch.Tensor] = None) -> None:
        """Chunked causal conv1d + SiLU over x [B, T, C] (replaces the torch
        F.conv1d prefill of braid/model/gdn.py:171-226). Equals conv1d_decode
        applied to each live token, bit for bit; pad positions write 0."""
        _check(conv_pool.is_cuda and conv_pool.dtype == torch.float32,
               "conv_pool must be cuda fp32")
        _check(conv_pool.is_contiguous(), "conv_pool must be contiguous")
        _check(slot_idx.dtype == torch.int32, "slot_idx must be int32")
        _check(slot_idx.is_cuda and slot_idx.is_contiguous(), "slot_idx must be contiguous cuda")
        _check(conv_pool.dim() == 3, "conv_pool must be [S_max, C, K]")
        n_slots, C, K = conv_pool.shape
        _check(x.dim() == 3 and x.size(2) == C, "x must be [B, T, C]")
        B, T = x.size(0), x.size(1)
        _check(tuple(out.shape) == (B, T, C), "out must be [B, T, C]")
        _check(tuple(weight.shape) == (C, K), "weight must be [C, K]")
        _check_dense_f32((weight,), "weight must be contiguous cuda fp32")
        _check(slot_idx.numel() == B, "slot_idx must have one entry per batch row")
        _check(x.dtype in _ACT_DTYPES,
               "x must be fp32 or bf16 (the activation dtypes braid runs)")
        _check(x.is_cuda and x.is_contiguous(), "x must be contiguous")
        _check(out.is_cuda and out.dtype == torch.float32 and out.is_contiguous(),
               "out must be contiguous fp32")
        bias_p = None
        if bias is not None and bias.numel() > 0:
            _check_dense_f32((bias,), "bias must be contiguous cuda fp32")
            _check(bias.numel() == C, "bias must be [C]")
            bias_p = _ptr(bias)
        if seq_lens is not None:
            _check(seq_lens.is_cuda and seq_lens.dtype == torch.int32
                   and seq_lens.is_contiguous(), "seq_lens must be contiguous cuda int32")
            _check(seq_lens.numel() == B, "seq_lens must have one entry per batch row")
        self._call("braid_conv1d_prefill", conv_pool.device, _ptr(conv_pool), n_slots, C, K,
                   _ptr(slot_idx), B, T, _ptr(x), _ACT_DTYPES[x.dtype], _ptr(weight), bias_p,
                   _ptr(out), _ptr(seq_lens))

    # -- FP8 activation quant ---------------------------------------------------

    def quantize_act(self, x: torch.Tensor) -> list:
        """x -> [q (float8_e4m3fn, x's shape), scale ([1, 1] fp32)]
        (quant_act.cu:140-176)."""
        _check(x.is_cuda, "x must be cuda")
        _check(x.is_contiguous(), "x must be contiguous")
        _check(x.dtype in _QUANT_DTYPES, "activation must be fp32, bf16 or fp16")
        n = x.numel()
        _check(n > 0, "x must not be empty")
        q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
        scale = torch.empty((1, 1), dtype=torch.float32, device=x.device)
        partial = torch.empty(self._lib.braid_quantize_act_workspace(n), dtype=torch.float32,
                              device=x.device)
        self._call("braid_quantize_act", x.device, _ptr(x), _QUANT_DTYPES[x.dtype], n,
                   _ptr(q), _ptr(scale), _ptr(partial))
        return [q, scale]

    def quantize_act_into(self, x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor) -> None:
        """quantize_act into caller-owned outputs, allocating nothing: q
        (float8_e4m3fn or uint8, x's element count) and scale (one fp32). The
        partial maxima live in the library's per-GPU device scratch, so calls
        that overlap on one GPU race (braid_quantize_act_noalloc)."""
        _check(x.is_cuda and q.is_cuda and scale.is_cuda, "x, q and scale must be cuda")
        _check(x.is_contiguous() and q.is_contiguous(), "x and q must be contiguous")
        _check(x.dtype in _QUANT_DTYPES, "activation must be fp32, bf16 or fp16")
        _check(q.dtype in (torch.float8_e4m3fn, torch.uint8) and q.numel() == x.numel(),
               "q must hold x's element count as float8_e4m3fn or uint8")
        _check(scale.dtype == torch.float32 and scale.numel() == 1, "scale must be one fp32")
        n = x.numel()
        _check(n > 0, "x must not be empty")
        self._call("braid_quantize_act_noalloc", x.device, _ptr(x), _QUANT_DTYPES[x.dtype], n,
                   _ptr(q), _ptr(scale))

    # -- gated RMSNorm readout (+ out_proj input quant) -------------------------

    def gated_rmsnorm(self, y: torch.Tensor, z: torch.Tensor, gamma: torch.Tensor,
                      eps: float, quantize: bool = True):
        """Readout of the scan (gdn.py:373-387 + norm.py:48-71), fused with the
        out_proj input quantization (quant.py:209-229).

        y: ``[..., H, HD]`` scan output (fp32, or already z's dtype); z: the gate,
        same element count, activation dtype; gamma ``[HD]`` fp32. Returns
        ``core`` shaped like z (z's dtype) and, with ``quantize``, ``q``
        (float8_e4m3fn, z's shape) and ``scale`` ([1, 1] fp32) as
        ``quantize_act(core)`` returns them.
        """
        _check(y.is_cuda and z.is_cuda and gamma.is_cuda, "y, z and gamma must be cuda")
        _check(z.dtype in _QUANT_DTYPES, "activation must be fp32, bf16 or fp16")
        _check(y.dtype in (torch.float32, z.dtype), "y must be fp32 or z's dtype")
        _check(y.is_contiguous() and z.is_contiguous(), "y and z must be contiguous")
        _check(gamma.dtype == torch.float32 and gamma.is_contiguous() and gamma.dim() == 1,
               "gamma must be a contiguous fp32 vector")
        HD = gamma.numel()
        _check(HD == 128, "only head_dim=128 is supported")
        _check(y.numel() == z.numel() and y.numel() % HD == 0,
               "y and z must hold the same number of head_dim rows")
        units = y.numel() // HD
        core = torch.empty(z.shape, dtype=z.dtype, device=z.device)
        q = scale = partial = None
        if quantize:
            _check(units > 0, "x must not be empty")
            q = torch.empty(z.shape, dtype=torch.float8_e4m3fn, device=z.device)
            scale = torch.empty((1, 1), dtype=torch.float32, device=z.device)
            partial = torch.empty(self._lib.braid_gated_rmsnorm_workspace(units),
                                  dtype=torch.float32, device=z.device)
        self._call("braid_gated_rmsnorm_quant", z.device, _ptr(y), _QUANT_DTYPES[y.dtype],
                   _ptr(z), _QUANT_DTYPES[z.dtype], _ptr(gamma), float(eps), units, HD,
                   _ptr(core), _ptr(q), _ptr(scale), _ptr(partial))
        return (core, q, scale) if quantize else core

    # -- FP8 GEMM (hipBLASLt) ------------------------------------------------------

    def _gemm_workspace(self, device: torch.device) -> torch.Tensor:
        """One workspace per device, allocated on first use (outside any graph
        capture, since the first call of a shape also selects its algorithm)."""
        key = torch.device(device).index or 0
        ws = self._workspaces.get(key)
        if ws is None:
            ws = torch.empty(self._lib.braid_fp8_gemm_workspace(), dtype=torch.uint8,
                             device=device)
            self._workspaces[key] = ws
        return ws

    def fp8_matmul(self, xq: torch.Tensor, sx: torch.Tensor, w: torch.Tensor,
                   sw: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """``torch._scaled_mm(xq, w.t(), scale_a=sx, scale_b=sw, out_dtype)``
        (braid/model/quant.py:232-241): xq [M, K] and w [N, K] float8_e4m3fn,
        sx / sw one-element fp32 dequant scales; returns [M, N]."""
        fp8 = torch.float8_e4m3fn
        _check(xq.is_cuda and w.is_cuda and sx.is_cuda and sw.is_cuda, "operands must be cuda")
        _check(xq.dtype == fp8 and w.dtype == fp8, "xq and w must be float8_e4m3fn")
        _check(xq.dim() == 2 and w.dim() == 2 and xq.size(1) == w.size(1),
               "xq must be [M, K] and w [N, K]")
        _check(xq.is_contiguous() and w.is_contiguous(), "xq and w must be contiguous")
        _check(sx.dtype == torch.float32 and sw.dtype == torch.float32
               and sx.numel() == 1 and sw.numel() == 1, "scales must be one fp32 element each")
        _check(out_dtype in _QUANT_DTYPES, "out dtype must be bf16, fp16 or fp32")
        M, K = xq.shape
        N = w.size(0)
        out = torch.empty(M, N, dtype=out_dtype, device=xq.device)
        ws = self._gemm_workspace(xq.device)
        self._call("braid_fp8_gemm", xq.device, _ptr(xq), _ptr(sx), _ptr(w), _ptr(sw), _ptr(out),
                   _QUANT_DTYPES[out_dtype], M, N, K, _ptr(ws), ws.numel())
        return out


@lru_cache(maxsize=1)
def load_gdn() -> GDNKernels:
    """Load the prebuilt gfx950 kernel library (no JIT; build with
    ``python -m braid_amd.build``)."""
    return GDNKernels(open_library())
