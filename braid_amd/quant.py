"""Dynamic per-tensor FP8 activation quantization, host side.

Mirrors ``braid.model.quant.quantize_act`` (braid/model/quant.py:209-229):
``[M, K]`` (any shape) -> (float8_e4m3fn codes, ``[1, 1]`` fp32 dequant scale),
bit-identical to ``(x.float() / scale).clamp(-448, 448).to(float8_e4m3fn)``
with ``scale = (x.float().abs().amax() / 448).clamp(min=1e-12)``.

The reference fell back to that torch spelling for a non-contiguous input.
Here a non-contiguous input is copied to a dense tensor and quantized by the
same kernel; the codes and scale depend only on the values, so the result is
the one the torch spelling gives. There is no torch or CPU fallback.
"""
from __future__ import annotations

import torch

from braid_amd.kernels.loader import load_gdn

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
EPS = 1e-12


def quantize_act(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if not x.is_contiguous():
        x = x.contiguous()
    q, scale = load_gdn().quantize_act(x)
    return q, scale
