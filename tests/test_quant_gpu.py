"""quantize_act on the GPU: bit-identical to torch's spelling on the same device
(reference tests/test_quant.py:391-477) and to the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from braid_amd.quant import quantize_act
from gpu_helpers import DEV, gen

pytestmark = pytest.mark.gpu
FP8_MAX, EPS = 448.0, 1e-12


def torch_spelling(x):
    """braid/model/quant.py:115 and :228-229."""
    scale = (x.float().abs().amax() / FP8_MAX).clamp(min=EPS).reshape(1, 1)
    return (x.float() / scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn), scale


def _bytes(q):
    return q.view(torch.uint8)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16],
                         ids=["bf16", "fp32", "fp16"])
@pytest.mark.parametrize("shape", [(1, 4096), (8, 4096), (37, 12288), (128, 12288), (3, 1001)],
                         ids=["m1", "m8", "m37", "m128", "ragged"])
def test_bit_identical_to_the_torch_spelling(kern, dt, shape):
    x = (torch.randn(*shape, generator=gen(17), device=DEV) * 3.5).to(dt)
    q, s = kern.quantize_act(x)
    qr, sr = torch_spelling(x)
    assert q.dtype == torch.float8_e4m3fn and tuple(q.shape) == shape and tuple(s.shape) == (1, 1)
    assert torch.equal(s, sr), f"scale {s.item():.9e} vs {sr.item():.9e}"
    diff = int((_bytes(q) != _bytes(qr)).sum())
    assert diff == 0, f"{diff} of {q.numel()} fp8 bytes differ"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_bit_identical_to_the_oracle(kern, dt):
    x = (torch.randn(64, 4096, generator=gen(3), device=DEV) * 2).to(dt)
    q, s = kern.quantize_act(x)
    qo, so = oracle.quantize_act(x.float().cpu().numpy())
    assert s.item() == float(so)
    assert np.array_equal(_bytes(q).cpu().numpy(), qo)


def test_degenerate_scales(kern):
    for label, x in (
        ("zeros", torch.zeros(4, 4096, device=DEV, dtype=torch.bfloat16)),
        ("huge", torch.full((4, 4096), 60000.0, device=DEV, dtype=torch.bfloat16)),
        ("tiny", torch.full((4, 4096), 1e-10, device=DEV, dtype=torch.bfloat16)),
    ):
        q, s = kern.quantize_act(x)
        qr, sr = torch_spelling(x)
        assert torch.isfinite(s).all(), label
        assert torch.equal(s, sr), label
        assert torch.equal(_bytes(q), _bytes(qr)), label


def test_a_nan_activation_survives_quantization(kern):
    x = torch.randn(4, 4096, generator=gen(3), device=DEV, dtype=torch.bfloat16)
    x[2, 100] = float("nan")
    q, s = kern.quantize_act(x)
    qr, sr = torch_spelling(x)
    assert torch.isnan(s).all() and torch.isnan(sr).all()
    assert torch.equal(_bytes(q), _bytes(qr))


def test_a_non_contiguous_activation_quantizes_as_its_contiguous_copy(kern):
    base = torch.randn(64, 4096, generator=gen(5), device=DEV, dtype=torch.bfloat16)
    view = base.t()
    assert not view.is_contiguous()
    with pytest.raises(RuntimeError, match="contiguous"):
        kern.quantize_act(view)
    q, s = quantize_act(view)
    qc, sc = kern.quantize_act(view.contiguous())
    assert torch.equal(s, sc) and torch.equal(_bytes(q), _bytes(qc))


def test_graph_replay_gives_the_eager_result(kern):
    x = torch.randn(64, 4096, generator=gen(8), device=DEV, dtype=torch.bfloat16)
    q_eager, s_eager = kern.quantize_act(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kern.quantize_act(x)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = kern.quantize_act(x)
    for i in range(3):
        x.normal_(generator=gen(100 + i))
        ref_q, ref_s = kern.quantize_act(x)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[1], ref_s) and torch.equal(_bytes(out[0]), _bytes(ref_q))
