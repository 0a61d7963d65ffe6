"""FP8 W8A8 host side: activation and weight quantization and the GEMM.

Mirrors braid/model/quant.py: ``quantize_act`` (:209-229), ``FP8Weight`` and
``quantize_weight`` (:91-154), ``fp8_matmul`` / ``fp8_linear`` / ``linear`` /
``project`` (:232-289). The quantizer is the library's two-launch kernel and
the GEMM is hipBLASLt through the library's ``braid_fp8_gemm``.

``quantize_act`` (braid/model/quant.py:209-229):
``[M, K]`` (any shape) -> (float8_e4m3fn codes, ``[1, 1]`` fp32 dequant scale),
bit-identical to ``(x.float() / scale).clamp(-448, 448).to(float8_e4m3fn)``
with ``scale = (x.float().abs().amax() / 448).clamp(min=1e-12)``.

The reference fell back to that torch spelling for a non-contiguous input.
Here a non-contiguous input is copied to a dense tensor and quantized by the
same kernel; the codes and scale depend only on the values, so the result is
the one the torch spelling gives. There is no torch or CPU fallback.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from braid_amd.kernels.loader import load_gdn

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
EPS = 1e-12


def quantize_act(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if not x.is_contiguous():
        x = x.contiguous()
    q, scale = load_gdn().quantize_act(x)
    return q, scale


@dataclass
class FP8Weight:
    """A ``[N, K]`` weight as fp8 codes with one ``[1, 1]`` fp32 dequant scale
    (braid/model/quant.py:91-106)."""

    data: torch.Tensor
    scale: torch.Tensor
    shape: tuple

    @property
    def nbytes(self) -> int:
        return self.data.numel() + 4


def quantize_weight(w: torch.Tensor) -> FP8Weight:
    """``[N, K]`` -> fp8 with one per-tensor scale, done once at load
    (braid/model/quant.py:134-154). The reference's scale,
    ``max(|amax|, |amin|) / 448`` clamped at 1e-12, is ``amax(|w|) * fl(1/448)``
    clamped, and its codes are ``(w / scale).clamp(-448, 448)`` cast to e4m3fn:
    exactly what ``quantize_act`` computes, so the same kernel quantizes
    weights (without the reference's fp32 image of the weight)."""
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got {tuple(w.shape)}")
    N, K = w.shape
    if K % 16 or N % 16:
        raise ValueError(
            f"_scaled_mm needs both weight dims to be multiples of 16; got [{N}, {K}]. "
            "Leave this projection in bf16.")
    data, scale = quantize_act(w)
    return FP8Weight(data=data, scale=scale, shape=(N, K))


def fp8_matmul(xq: torch.Tensor, sx: torch.Tensor, w: FP8Weight,
               out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The GEMM alone on an already-quantized ``[M, K]`` activation
    (braid/model/quant.py:232-241)."""
    return load_gdn().fp8_matmul(xq, sx, w.data, w.scale, out_dtype)


def fp8_linear(x: torch.Tensor, w: FP8Weight) -> torch.Tensor:
    """``F.linear(x, w)`` for one call site; leading dims are kept
    (braid/model/quant.py:244-252)."""
    *lead, K = x.shape
    xq, sx = quantize_act(x.reshape(-1, K))
    return fp8_matmul(xq, sx, w, out_dtype=x.dtype).reshape(*lead, w.shape[0])


def linear(x: torch.Tensor, w) -> torch.Tensor:
    """Dispatch on the weight's type (braid/model/quant.py:255-257)."""
    return fp8_linear(x, w) if isinstance(w, FP8Weight) else F.linear(x, w)


def project(x: torch.Tensor, *weights) -> list:
    """Several projections of one activation, quantized ONCE for all the FP8
    ones (braid/model/quant.py:260-289)."""
    if not any(isinstance(w, FP8Weight) for w in weights):
        return [F.linear(x, w) for w in weights]
    *lead, K = x.shape
    xq, sx = quantize_act(x.reshape(-1, K))
    out = []
    for w in weights:
        if isinstance(w, FP8Weight):
            out.append(fp8_matmul(xq, sx, w, out_dtype=x.dtype).reshape(*lead, w.shape[0]))
        else:
            out.append(F.linear(x, w))
    return out
