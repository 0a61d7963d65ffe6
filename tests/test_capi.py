"""The C-ABI library on the CPU: it loads, exports every symbol the header
declares, and rejects bad arguments before touching a GPU.

No compute call is made here (there is no GPU in the build container); the
error paths exercised return before any HIP call.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from braid_amd.kernels import loader

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "braid_gdn.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(braid_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not loader.LIB_PATH.exists():
        from braid_amd.build import build
        build()
    return loader.open_library()


def test_header_declares_the_six_reference_entry_points():
    names = _declared()
    for fn in ("braid_gdn_decode", "braid_gdn_decode_raw", "braid_gdn_prefill",
               "braid_gdn_prefill_raw", "braid_conv1d_decode", "braid_quantize_act"):
        assert fn in names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(_declared()) == set(loader.SIGNATURES), "ctypes prototypes out of sync with header"
    assert lib.braid_abi_version() == 1


def _err(lib) -> str:
    return lib.braid_last_error().decode()


def test_decode_rejects_bad_shapes_before_any_gpu_call(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: every case fails host-side
    rc = lib.braid_gdn_decode(fake, 1, 160, 32, 16, 64, 128, fake, 4, fake, 2048, fake, 2048,
                              fake, 4096, fake, fake, fake, None)
    assert rc == 1 and "only SS=HD=128" in _err(lib)
    rc = lib.braid_gdn_decode(fake, 7, 160, 32, 16, 128, 128, fake, 4, fake, 2048, fake, 2048,
                              fake, 4096, fake, fake, fake, None)
    assert rc == 1 and "fp32, fp16 or bf16" in _err(lib)
    rc = lib.braid_gdn_decode(fake, 1, 160, 32, 12, 128, 128, fake, 4, fake, 2048, fake, 2048,
                              fake, 4096, fake, fake, fake, None)
    assert rc == 1 and "divisible" in _err(lib)
    rc = lib.braid_gdn_decode(fake, 1, 160, 32, 16, 128, 128, fake, 4, fake, 1000, fake, 2048,
                              fake, 4096, fake, fake, fake, None)
    assert rc == 1 and "rows overlap" in _err(lib)


def test_zero_batch_is_a_no_op(lib):
    fake = ctypes.c_void_p(4096)
    rc = lib.braid_gdn_decode(fake, 1, 160, 32, 16, 128, 128, fake, 0, None, 0, None, 0,
                              None, 0, None, None, None, None)
    assert rc == 0 and _err(lib) == ""


def test_raw_and_conv_and_quant_reject_bad_arguments(lib):
    fake = ctypes.c_void_p(4096)
    rc = lib.braid_gdn_decode_raw(fake, 1, 8, 4, 2, 128, 128, fake, 2, fake, 256, fake, 256,
                                  fake, 512, fake, fake, 1, fake, fake, fake, None)
    assert rc == 1 and "fp32 or bf16" in _err(lib)
    rc = lib.braid_conv1d_decode(fake, 8, 512, 5, fake, 2, fake, 0, fake, None, fake, None)
    assert rc == 1 and "not instantiated" in _err(lib)
    rc = lib.braid_conv1d_decode(fake, 8, 512, 4, fake, 2, fake, 1, fake, None, fake, None)
    assert rc == 1 and "fp32 or bf16" in _err(lib)
    rc = lib.braid_quantize_act(fake, 2, 0, fake, fake, fake, None)
    assert rc == 1 and "empty" in _err(lib)
    rc = lib.braid_quantize_act(fake, 9, 16, fake, fake, fake, None)
    assert rc == 1 and "fp32, bf16 or fp16" in _err(lib)
    assert lib.braid_quantize_act_workspace(64 * 4096) == 128
    assert lib.braid_quantize_act_workspace(10 ** 9) == 1024


def test_prefill_rejects_negative_t(lib):
    fake = ctypes.c_void_p(4096)
    rc = lib.braid_gdn_prefill(fake, 0, 8, 4, 2, 128, 128, fake, 2, -1, fake, fake, fake,
                               fake, fake, fake, None)
    assert rc == 1 and "non-negative" in _err(lib)


# --- the torch-facing shim: checks that fire before the library is called -----

def _shim():
    return loader.GDNKernels.__new__(loader.GDNKernels)


def test_shim_refuses_cpu_tensors_and_bad_dtypes():
    k = _shim()
    pool = torch.zeros(4, 2, 128, 128)
    slots = torch.zeros(1, dtype=torch.int32)
    q = torch.zeros(1, 1, 128)
    with pytest.raises(RuntimeError, match="pool must be cuda"):
        k.gdn_decode(pool, slots, q, q, torch.zeros(1, 2, 128), torch.zeros(1, 2),
                     torch.zeros(1, 2), torch.zeros(1, 2, 128))
    with pytest.raises(RuntimeError, match="x must be cuda"):
        k.quantize_act(torch.zeros(4, 4))
    with pytest.raises(RuntimeError, match="conv_pool must be cuda fp32"):
        k.conv1d_decode(torch.zeros(2, 8, 4), slots, torch.zeros(1, 8), torch.zeros(8, 4),
                        None, torch.zeros(1, 8))


def test_row_stride_rules_match_the_reference():
    buf = torch.zeros(3, 8192)
    q = buf[:, :2048].unflatten(-1, (16, 128))
    assert loader._row_stride_3d(q, "q", require_cuda=False) == 8192
    with pytest.raises(RuntimeError, match="rows overlap"):
        loader._row_stride_3d(torch.zeros(4, 2, 128).as_strided((4, 2, 128), (128, 128, 1)), "q",
                              require_cuda=False)
    with pytest.raises(RuntimeError, match="dense in its last two dims"):
        loader._row_stride_3d(torch.zeros(2, 128, 2).transpose(1, 2), "q", require_cuda=False)


def test_added_entry_points_reject_bad_arguments_before_any_gpu_call(lib):
    fake = ctypes.c_void_p(4096)
    rc = lib.braid_gated_rmsnorm_quant(fake, 0, fake, 2, fake, ctypes.c_float(1e-6), 64, 64,
                                       fake, None, None, None, None)
    assert rc == 1 and "head_dim must be 128" in _err(lib)
    rc = lib.braid_gated_rmsnorm_quant(fake, 0, fake, 2, fake, ctypes.c_float(1e-6), 64, 128,
                                       fake, fake, None, None, None)
    assert rc == 1 and "given together" in _err(lib)
    rc = lib.braid_gated_rmsnorm_quant(fake, 0, fake, 2, fake, ctypes.c_float(1e-6), 0, 128,
                                       fake, fake, fake, fake, None)
    assert rc == 1 and "must not be empty" in _err(lib)
    rc = lib.braid_gdn_conv_decode_raw(fake, 1, 16, 8, 4, 128, 128, fake, 3, fake, 2, fake, 2,
                                       fake, None, fake, fake, 2, fake, fake, fake, None)
    assert rc == 1 and "conv_kernel == 4" in _err(lib)
    rc = lib.braid_gdn_conv_decode_raw(fake, 1, 16, 8, 2, 128, 128, fake, 4, fake, 2, fake, 2,
                                       fake, None, fake, fake, 2, fake, fake, fake, None)
    assert rc == 1 and "1 or 2 value heads" in _err(lib)
    rc = lib.braid_fp8_gemm(fake, fake, fake, fake, fake, 2, 4, 24, 40, fake,
                            lib.braid_fp8_gemm_workspace(), None)
    assert rc == 1 and "multiples of 16" in _err(lib)
    rc = lib.braid_fp8_gemm(fake, fake, fake, fake, fake, 2, 0, 32, 32, fake, 0, None)
    assert rc == 1 and "positive" in _err(lib)
    assert lib.braid_fp8_gemm_workspace() == 32 << 20
    assert lib.braid_gated_rmsnorm_workspace(64 * 32) == 256


def test_stream_probe_library_loads_and_rejects_bad_arguments():
    """libbraid_probe.so (bench.py's roofline ceiling, outside the drop-in
    ABI) exports braid_probe_stream and refuses bad arguments before any GPU
    call."""
    import ctypes

    from braid_amd.build import PROBE_LIB

    if not PROBE_LIB.exists():
        pytest.skip("libbraid_probe.so not built")
    lib = ctypes.CDLL(str(PROBE_LIB))
    fn = lib.braid_probe_stream
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    dummy = ctypes.c_void_p(16)
    assert fn(0, None, 4, dummy, None, None) != 0      # null base
    assert fn(0, dummy, 0, dummy, None, None) != 0     # no tiles
    assert fn(3, dummy, 4, dummy, None, None) != 0     # unknown kind
    assert fn(1, dummy, 4, dummy, None, None) != 0     # read pass without a sink


def test_host_prefill_plan_picks_the_measured_plans(lib):
    """braid_prefill_plan: the tiers an eager ragged prefill runs (n8 eighth
    rows, n4 quarter rows, n2 split rows; returned as n8 * 2^20 + n4 * 2^10 +
    n2), chosen by simulating the
    launch on 256 CUs of two workgroup slots. The expected plans are the
    choices that measured within a few percent of the best of every plan
    timed on MI355X (H = 32); they pin the simulation, the cost table and the
    tie order."""
    cases = {
        (454, 610, 334, 542, 393, 861, 814, 65): (0, 1, 6),   # config 2
        (1003, 300, 1001, 383): (0, 3, 1),
        (900, 850, 200, 200, 200, 200, 200, 200): (0, 2, 2),
        (1024,) + (128,) * 15: (1, 0, 0),
        (256,) * 16: (0, 0, 0),
    }
    for lens, plan in cases.items():
        arr = (ctypes.c_int32 * len(lens))(*lens)
        p = lib.braid_prefill_plan(arr, len(lens), max(lens), 32, 256)
        assert (p >> 20, (p >> 10) & 1023, p & 1023) == plan, lens
    # one row: the eighth layout; a batch of empty rows plans nothing
    one = (ctypes.c_int32 * 1)(700)
    assert lib.braid_prefill_plan(one, 1, 700, 32, 256) == 1 << 20
    zeros = (ctypes.c_int32 * 3)(0, 0, 0)
    assert lib.braid_prefill_plan(zeros, 3, 10, 32, 256) == 0
    assert lib.braid_prefill_plan(None, 3, 10, 32, 256) == -1
    assert "host lengths" in _err(lib)


def _plan(lib, lens, T=None, H=32, cus=256):
    arr = (ctypes.c_int32 * len(lens))(*lens)
    p = lib.braid_prefill_plan(arr, len(lens), T if T is not None else max(max(lens), 1), H, cus)
    assert p >= 0, _err(lib)
    return p >> 20, (p >> 10) & 1023, p & 1023


def test_host_prefill_plan_edge_cases(lib):
    """The host planner's invariants, away from the measured batches: a plan
    never upgrades more rows than it has live ones (or more than its tier
    limits: n8 <= 2, n4 <= 6, n2 <= 8); it depends only on the multiset of
    live lengths (order and lengths clipped to T); a single live row among
    empty ones runs the eighth layout, as a batch of one does; all-equal rows
    at every CU's two slots plan nothing; B at the planned kernel's row cap
    (1024) plans in bounded host time."""
    import random
    import time

    rng = random.Random(7)
    for _ in range(40):
        B = rng.randint(1, 40)
        lens = [rng.choice([0, rng.randint(1, 1024)]) for _ in range(B)]
        n8, n4, n2 = _plan(lib, lens, T=1024)
        live = sum(1 for x in lens if x > 0)
        assert n8 <= 2 and n4 <= 6 and n2 <= 8
        assert n8 + n4 + n2 <= max(live, 0) or (live == 0 and (n8, n4, n2) == (0, 0, 0)), lens
        shuffled = lens[:]
        rng.shuffle(shuffled)
        assert _plan(lib, shuffled, T=1024) == (n8, n4, n2)
    # clipping to T: lengths beyond T plan as T
    assert _plan(lib, [5000, 300], T=1000) == _plan(lib, [1000, 300], T=1000)
    # one live row among empty ones: the same as that row alone
    assert _plan(lib, [0, 0, 700, 0]) == _plan(lib, [700]) == (1, 0, 0)
    # sixteen equal rows fill 512 workgroup slots whole: nothing to upgrade
    assert _plan(lib, [256] * 16) == (0, 0, 0)
    # the row cap: 1024 rows, distinct lengths (no cache hit), bounded time
    lens = [1 + (i * 37) % 97 for i in range(1024)]
    t0 = time.perf_counter()
    n8, n4, n2 = _plan(lib, lens)
    assert time.perf_counter() - t0 < 2.0
    assert n8 <= 2 and n4 <= 6 and n2 <= 8


def test_host_prefill_plan_cache_evicts_one_at_a_time(lib):
    """Past its bound (4096 length sets) the plan cache evicts its oldest
    entries, not everything: plans stay what the simulation gives for any
    history of calls."""
    first = _plan(lib, [454, 610, 334, 542, 393, 861, 814, 65])
    for i in range(4200):
        _plan(lib, [100 + i % 900, 50 + i // 900, 7], T=2048)
    assert _plan(lib, [454, 610, 334, 542, 393, 861, 814, 65]) == first == (0, 1, 6)


def test_launch_knobs_ignore_malformed_environment_values():
    """A launch knob's environment value counts only when it is a whole
    decimal number in [0, 2^30]; anything else leaves the knob unset (-1), so
    a typo cannot force a launch shape. Checked in a fresh process, since the
    knobs are read once when the library loads."""
    import os
    import subprocess
    import sys

    code = (
        "import ctypes, sys; from braid_amd.kernels import loader; "
        "lib = ctypes.CDLL(str(loader.LIB_PATH)); "
        "print(' '.join(str(lib.braid_get_launch_override(i)) for i in range(6)))"
    )
    env = dict(os.environ, BRAID_DECODE_XCD_REMAP="abc", BRAID_DECODE_WGS_PER_CU="2x",
               BRAID_PREFILL_COLS="", BRAID_DECODE_PARTS="-2", BRAID_PREFILL_PLAN="1025",
               BRAID_FP8_GEMM="0")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         cwd=str(Path(__file__).resolve().parents[1]), check=True)
    assert out.stdout.split() == ["-1", "-1", "-1", "-1", "1025", "0"], out.stdout + out.stderr
