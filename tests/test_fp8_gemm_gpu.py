"""FP8 W8A8 GEMM (braid_fp8_gemm: the streaming kernel at decode shapes,
hipBLASLt otherwise) on the GPU.

Reference: braid/model/quant.py:232-289 (fp8_matmul = torch._scaled_mm with
per-tensor scales; fp8_linear / project quantize the activation once).
The FP8 products are exact in fp32 and only the accumulation order is the
kernel's, so the output is checked against an fp32 reference of the same
dequantized operands: within one unit of the output dtype's rounding plus a
fp32 accumulation allowance, on both paths (the launch knob forces
hipBLASLt). It is also checked against torch._scaled_mm on this device, the
reference's own call.
"""
from __future__ import annotations

import pytest
import torch

from braid_amd.quant import (FP8Weight, fp8_linear, fp8_matmul, linear, project,
                             quantize_act, quantize_weight)
from braid_amd.kernels.loader import load_gdn
from gpu_helpers import DEV, gen

pytestmark = pytest.mark.gpu
EPS_OUT = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -23}


def _ref(xq, sx, w: FP8Weight):
    return (xq.float() * sx) @ (w.data.float() * w.scale).t()


def _check(out, ref, dt, K):
    # rounding of the output (half an ulp, relative) + fp32 accumulation over K terms
    mag = ref.abs()
    tol = mag * EPS_OUT[dt] + 1e-6 * K ** 0.5 * (mag.max() + 1e-30)
    err = (out.float() - ref).abs()
    assert bool((err <= tol).all()), f"max excess {(err - tol).max().item():.3e}"


PATHS = {"default": None, "hipblaslt": 0}


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (64, 12288, 4096), (37, 4096, 4096),
                                   (64, 4096, 4096), (128, 1024, 2048)])
def test_matches_the_fp32_reference(M, N, K, dt, path):
    x = torch.randn(M, K, generator=gen(M + N), device=DEV).to(dt)
    w = quantize_weight(torch.randn(N, K, generator=gen(K), device=DEV) * 0.02)
    xq, sx = quantize_act(x)
    with load_gdn().launch_override(fp8_gemm=PATHS[path]):
        out = fp8_matmul(xq, sx, w, out_dtype=dt)
    assert out.dtype == dt and tuple(out.shape) == (M, N)
    _check(out, _ref(xq, sx, w), dt, K)


# the streaming kernel's edges: one workgroup (N = 16), every partial 16-row
# block (M = 17, 33, 49), 1 and 16 k-steps per wave (K = 1024, 16384), a
# column count that is no multiple of 48 or 32; and shapes it leaves to
# hipBLASLt (M = 65; K not 1024 * 2^i)
@pytest.mark.parametrize("M,N,K", [(1, 16, 1024), (17, 48, 2048), (33, 4112, 1024),
                                   (49, 1024, 16384), (64, 272, 8192), (65, 512, 1024),
                                   (8, 512, 3072)])
def test_stream_kernel_edges(M, N, K):
    x = torch.randn(M, K, generator=gen(3 * M + N), device=DEV).bfloat16()
    w = quantize_weight(torch.randn(N, K, generator=gen(K + 1), device=DEV) * 0.02)
    xq, sx = quantize_act(x)
    for dt in (torch.bfloat16, torch.float32):
        _check(fp8_matmul(xq, sx, w, out_dtype=dt), _ref(xq, sx, w), dt, K)


def test_stream_kernel_is_deterministic_and_agrees_with_hipblaslt():
    x = torch.randn(64, 4096, generator=gen(21), device=DEV).bfloat16()
    w = quantize_weight(torch.randn(12288, 4096, generator=gen(22), device=DEV) * 0.02)
    xq, sx = quantize_act(x)
    a = fp8_matmul(xq, sx, w, out_dtype=torch.float32)
    b = fp8_matmul(xq, sx, w, out_dtype=torch.float32)
    assert torch.equal(a, b)
    with load_gdn().launch_override(fp8_gemm=0):
        lib = fp8_matmul(xq, sx, w, out_dtype=torch.float32)
    # two fp32 summation orders of the same exact products
    assert bool(((a - lib).abs() <= 1e-5 * a.abs().max()).all())


@pytest.mark.parametrize("M,N,K", [(16, 4096, 4096), (64, 12288, 4096)])
def test_agrees_with_torch_scaled_mm(M, N, K):
    x = torch.randn(M, K, generator=gen(5), device=DEV).bfloat16()
    w = quantize_weight(torch.randn(N, K, generator=gen(6), device=DEV) * 0.02)
    xq, sx = quantize_act(x)
    ours = fp8_matmul(xq, sx, w)
    theirs = torch._scaled_mm(xq, w.data.t(), scale_a=sx, scale_b=w.scale,
                              out_dtype=torch.bfloat16)
    # both round one fp32 sum to bf16; orders may differ, so allow one bf16 ulp
    diff = (ours.float() - theirs.float()).abs()
    assert bool((diff <= theirs.float().abs() * 2.0 ** -7 + 1e-6).all())
    assert (diff == 0).float().mean().item() > 0.9


def test_weight_quantization_is_the_reference_spelling():
    w = torch.randn(256, 512, generator=gen(7), device=DEV).bfloat16() * 0.05
    fw = quantize_weight(w)
    t = w.detach()
    scale = ((torch.maximum(t.amax().abs(), t.amin().abs()).float() / 448.0)
             .clamp(min=1e-12).reshape(1, 1))
    codes = (w.float() / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    assert torch.equal(fw.scale, scale)
    assert torch.equal(fw.data.view(torch.uint8), codes.view(torch.uint8))
    with pytest.raises(ValueError, match="multiples of 16"):
        quantize_weight(torch.randn(24, 40, device=DEV))


def test_linear_and_project_quantize_once_and_keep_leading_dims():
    x = torch.randn(4, 3, 1024, generator=gen(8), device=DEV).bfloat16()
    w1 = quantize_weight(torch.randn(2048, 1024, generator=gen(9), device=DEV) * 0.02)
    w2 = quantize_weight(torch.randn(512, 1024, generator=gen(10), device=DEV) * 0.02)
    wb = (torch.randn(256, 1024, generator=gen(11), device=DEV) * 0.02).bfloat16()
    a, b, c = project(x, w1, w2, wb)
    assert a.shape == (4, 3, 2048) and b.shape == (4, 3, 512) and c.shape == (4, 3, 256)
    assert torch.equal(a, fp8_linear(x, w1)) and torch.equal(a, linear(x, w1))
    assert torch.equal(c, linear(x, wb))


def test_graph_replay_equals_eager():
    x = torch.randn(64, 4096, generator=gen(12), device=DEV).bfloat16()
    w = quantize_weight(torch.randn(4096, 4096, generator=gen(13), device=DEV) * 0.02)
    xq, sx = quantize_act(x)
    eager = fp8_matmul(xq, sx, w)            # also selects the algorithm
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fp8_matmul(xq, sx, w)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_argument_checks():
    from braid_amd.kernels.loader import load_gdn
    kern = load_gdn()
    xq = torch.zeros(4, 40, device=DEV).to(torch.float8_e4m3fn)
    w = torch.zeros(16, 40, device=DEV).to(torch.float8_e4m3fn)
    s = torch.ones(1, 1, device=DEV)
    with pytest.raises(RuntimeError, match="multiples of 16"):
        kern.fp8_matmul(xq, s, w, s)
    with pytest.raises(RuntimeError, match=r"\[M, K\]"):
        kern.fp8_matmul(xq, s, torch.zeros(16, 32, device=DEV).to(torch.float8_e4m3fn), s)
