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


def _fp8_values():
    """Every non-negative finite e4m3fn value, ascending (codes 0..126)."""
    return np.array(sorted(float(torch.tensor([c], dtype=torch.uint8)
                                 .view(torch.float8_e4m3fn).float().item())
                           for c in range(127)), dtype=np.float32)


@pytest.mark.parametrize("k", [0, -3, 5])
def test_exact_ties_and_their_neighbours_round_like_torch(kern, k):
    """Adversarial inputs for the quantizer's finite-scale path (a corrected
    reciprocal multiply and the hardware e4m3fn conversion): amax is chosen so
    that the scale amax * fl(1/448) is exactly 2^k. x / scale is then exact,
    and x holds every e4m3fn value, every midpoint between neighbours (where
    round-to-nearest-even decides), and the fp32 neighbours of both, times
    2^k, in both signs. Codes and scale must be torch's and the oracle's, bit
    for bit."""
    inv = np.float32(1.0 / 448.0)
    target = np.float32(2.0 ** k)
    a = np.float32(448.0 * 2.0 ** k)
    for _ in range(400):                 # nearest amax whose scale is exactly 2^k
        if np.float32(a * inv) == target:
            break
        a = np.nextafter(a, np.float32(np.inf) if np.float32(a * inv) < target
                         else np.float32(0), dtype=np.float32)
    assert np.float32(a * inv) == target
    v = _fp8_values()
    mids = ((v[:-1].astype(np.float64) + v[1:]) / 2).astype(np.float32)
    base = np.concatenate([v, mids])
    near = np.concatenate([base, np.nextafter(base, np.float32(np.inf)),
                           np.nextafter(base, np.float32(0))]) * target
    near = near[np.abs(near) <= a]
    x = np.concatenate([near, -near, [a]]).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV).reshape(1, -1)
    q, s = kern.quantize_act(xt)
    qr, sr = torch_spelling(xt)
    assert s.item() == float(target) and torch.equal(s, sr)
    diff = int((_bytes(q) != _bytes(qr)).sum())
    assert diff == 0, f"{diff} of {x.size} codes differ from torch"
    qo, so = oracle.quantize_act(x.reshape(1, -1))
    assert np.array_equal(_bytes(q).cpu().numpy().reshape(-1), qo.reshape(-1))


def _amax_for_scale(target):
    inv = np.float32(1.0 / 448.0)
    a = np.float32(448.0) * np.float32(target)
    for _ in range(400):
        if np.float32(a * inv) == target:
            return a
        a = np.nextafter(a, np.float32(np.inf) if np.float32(a * inv) < target
                         else np.float32(0), dtype=np.float32)
    raise AssertionError("no amax gives the scale exactly")


def test_every_fp32_value_at_unit_scale_encodes_like_torch(kern):
    """At a scale of exactly 1 the quotient is x itself, so this covers the
    e4m3fn conversion for every fp32 bit pattern with |x| <= amax (~2.3e9
    values, both signs, subnormals included), in chunks that each also hold
    amax. Codes must equal torch's spelling byte for byte."""
    a = _amax_for_scale(np.float32(1.0))
    a_bits = int(np.array([a], dtype=np.float32).view(np.int32)[0])
    chunk = 1 << 26
    amax_t = torch.tensor([a], device=DEV)
    for start in range(0, a_bits + 1, chunk):
        n = min(chunk, a_bits + 1 - start)
        bits = torch.arange(start, start + n, device=DEV, dtype=torch.int32)
        for sign in (0, -2 ** 31):
            x = torch.cat([(bits | sign).view(torch.float32), amax_t]).reshape(1, -1)
            q, s = kern.quantize_act(x)
            qr, sr = torch_spelling(x)
            assert s.item() == 1.0 and torch.equal(s, sr)
            diff = int((_bytes(q) != _bytes(qr)).sum())
            assert diff == 0, f"chunk at {start:#x} sign {sign}: {diff} codes differ"


def test_every_bf16_value_under_many_scales_encodes_like_torch(kern):
    """The finite-scale path divides by a corrected reciprocal multiply; this
    checks it against torch's true division for every bf16 value with
    |x| <= amax, under 512 scales whose amax spans the whole fp32 exponent
    range (scales below 1e-12 clamp to it), with amax itself in each tensor."""
    rng = np.random.default_rng(31)
    every = torch.arange(0, 1 << 16, device=DEV, dtype=torch.int32).to(torch.int16)
    xs = every.view(torch.bfloat16).float()
    xs = xs[torch.isfinite(xs)]
    exps = rng.integers(1, 255, 512)
    mants = rng.integers(0, 1 << 23, 512)
    for e, m in zip(exps, mants):
        a = np.array([(int(e) << 23) | int(m)], dtype=np.int32).view(np.float32)[0]
        a_t = torch.tensor([a], device=DEV)
        x = torch.cat([xs[xs.abs() <= a_t], a_t]).reshape(1, -1)
        q, s = kern.quantize_act(x)
        qr, sr = torch_spelling(x)
        assert torch.equal(s, sr), a
        diff = int((_bytes(q) != _bytes(qr)).sum())
        assert diff == 0, f"amax {a!r}: {diff} codes differ"
