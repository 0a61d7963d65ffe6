"""braid_quantize_act_noalloc: the allocation-free variant of quantize_act.

It keeps the pass-1 partial maxima in the library's own per-GPU device
scratch instead of a caller workspace. Called through the C ABI (ctypes) and
checked against braid_quantize_act on the same input: FP8 codes and scale
bit for bit, on two calls in a row, the second with a smaller input (the
scratch then still holds the first call's partials), in both orders of the
activation dtypes, and with graph capture.
"""
from __future__ import annotations

import pytest
import torch

from braid_amd.kernels import loader
from gpu_helpers import DEV, gen

pytestmark = pytest.mark.gpu
DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return loader.open_library()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _with_workspace(lib, x):
    n = x.numel()
    q = torch.empty(n, dtype=torch.uint8, device=DEV)
    s = torch.empty(1, dtype=torch.float32, device=DEV)
    part = torch.empty(lib.braid_quantize_act_workspace(n), dtype=torch.float32, device=DEV)
    rc = lib.braid_quantize_act(x.data_ptr(), DT[x.dtype], n, q.data_ptr(), s.data_ptr(),
                                part.data_ptr(), _stream())
    assert rc == 0, lib.braid_last_error().decode()
    return q, s


def _noalloc(lib, x, q=None, s=None):
    n = x.numel()
    q = torch.empty(n, dtype=torch.uint8, device=DEV) if q is None else q
    s = torch.empty(1, dtype=torch.float32, device=DEV) if s is None else s
    rc = lib.braid_quantize_act_noalloc(x.data_ptr(), DT[x.dtype], n, q.data_ptr(),
                                        s.data_ptr(), _stream())
    assert rc == 0, lib.braid_last_error().decode()
    return q, s


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16],
                         ids=["bf16", "fp32", "fp16"])
def test_noalloc_equals_the_workspace_entry_on_two_calls(lib, dt):
    big = (torch.randn(128, 12288, generator=gen(41), device=DEV) * 7.0).to(dt)
    small = (torch.randn(3, 1001, generator=gen(42), device=DEV) * 0.01).to(dt)
    for x in (big, small):  # the second call is smaller: stale partials must not leak in
        q0, s0 = _with_workspace(lib, x)
        q1, s1 = _noalloc(lib, x)
        torch.cuda.synchronize()
        print(f"{dt} n={x.numel()} scale {s1.item():.9e} ref {s0.item():.9e}", flush=True)
        assert torch.equal(s1, s0)
        assert torch.equal(q1, q0), f"{int((q1 != q0).sum())} of {q0.numel()} codes differ"


def test_noalloc_propagates_nan_and_then_recovers(lib):
    x = torch.randn(64, 4096, generator=gen(43), device=DEV).to(torch.bfloat16)
    x[5, 7] = float("nan")
    _, s = _noalloc(lib, x)
    torch.cuda.synchronize()
    assert s.isnan().all()
    y = torch.randn(8, 4096, generator=gen(44), device=DEV).to(torch.bfloat16)
    q1, s1 = _noalloc(lib, y)
    q0, s0 = _with_workspace(lib, y)
    torch.cuda.synchronize()
    assert torch.equal(s1, s0) and torch.equal(q1, q0)


def test_noalloc_replays_inside_a_graph(lib):
    x = (torch.randn(64, 4096, generator=gen(45), device=DEV) * 2).to(torch.bfloat16)
    q = torch.empty(x.numel(), dtype=torch.uint8, device=DEV)
    s = torch.empty(1, dtype=torch.float32, device=DEV)
    _noalloc(lib, x, q, s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _noalloc(lib, x, q, s)
    for seed in (46, 47, 48):
        x.copy_((torch.randn(64, 4096, generator=gen(seed), device=DEV) * seed).to(x.dtype))
        _with_workspace(lib, x[:1])  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        q0, s0 = _with_workspace(lib, x)
        torch.cuda.synchronize()
        assert torch.equal(s, s0) and torch.equal(q, q0), seed


def test_noalloc_rejects_bad_arguments(lib):
    x = torch.ones(16, device=DEV)
    q = torch.empty(16, dtype=torch.uint8, device=DEV)
    s = torch.empty(1, device=DEV)
    rc = lib.braid_quantize_act_noalloc(x.data_ptr(), 0, 0, q.data_ptr(), s.data_ptr(), None)
    assert rc == 1 and "must not be empty" in lib.braid_last_error().decode()
    rc = lib.braid_quantize_act_noalloc(x.data_ptr(), 9, 16, q.data_ptr(), s.data_ptr(), None)
    assert rc == 1 and "fp32, bf16 or fp16" in lib.braid_last_error().decode()
    rc = lib.braid_quantize_act_noalloc(None, 0, 16, q.data_ptr(), s.data_ptr(), None)
    assert rc == 1 and "non-null" in lib.braid_last_error().decode()


def test_loader_front_end_writes_caller_outputs(lib, kern):
    x = (torch.randn(16, 4096, generator=gen(49), device=DEV) * 3).to(torch.float16)
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(1, dtype=torch.float32, device=DEV)
    kern.quantize_act_into(x, q, s)
    q0, s0 = kern.quantize_act(x)
    torch.cuda.synchronize()
    assert torch.equal(s, s0.reshape(1)) and torch.equal(q.view(torch.uint8), q0.view(torch.uint8))
