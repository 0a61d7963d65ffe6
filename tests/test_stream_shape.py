"""The decode's launch shape (braid_amd/csrc/stream_shape.h) over device
topologies, on the CPU: a host-only program compiled with hipcc calls
stream_shape() with synthetic DeviceTopo values (no HIP runtime call), so a
partitioned device or an unknown one can be checked without the hardware.

A large launch (>= 6 tiles per CU for 16-bit tiles, 12 for fp32) takes the
two-per-CU residency cap, the device's LDS per CU halved, less the kernel's
own LDS and 1 KiB, at most 64 KiB, and, only on a device with 8 XCDs and a
tile count divisible by 8, the XCD-contiguous order (per = tiles / 8)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from braid_amd import build as B

PROGRAM = r"""
#include "stream_shape.h"
#include <cstdio>
int main() {
  using namespace braid;
  auto show = [](const char* name, StreamShape s) {
    std::printf("%s %d %zu\n", name, s.xcd_per, s.lds_pad);
  };
  const DeviceTopo full{256, 8, 160 * 1024}, cpx{32, 1, 160 * 1024}, small_lds{256, 8, 64 * 1024},
      unknown{};
  show("full_b128", stream_shape(4096, full, true, 8704));
  show("full_b64", stream_shape(2048, full, true, 8704));
  show("full_b48", stream_shape(1536, full, true, 8704));
  show("full_b40", stream_shape(1280, full, true, 8704));
  show("full_b32", stream_shape(1024, full, true, 8704));
  show("full_f32_b64", stream_shape(2048, full, false, 8704));
  show("full_f32_b96", stream_shape(3072, full, false, 8704));
  show("full_odd", stream_shape(4100, full, true, 8704));
  show("cpx_b16", stream_shape(512, cpx, true, 8704));
  show("small_lds", stream_shape(4096, small_lds, true, 8704));
  show("unknown", stream_shape(4096, unknown, true, 8704));
  show("override_remap_cap3", stream_shape(1024, full, true, 8704, 1, 3));
  show("override_off", stream_shape(4096, full, true, 8704, 0, 0));
  return 0;
}
"""


@pytest.fixture(scope="module")
def shapes(tmp_path_factory):
    hipcc = B.hipcc()
    if not shutil.which(hipcc) and not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("stream_shape")
    (d / "t.cpp").write_text(PROGRAM)
    exe = d / "t"
    subprocess.run([hipcc, "-x", "hip", "-std=c++17", "-I", str(B.CSRC), str(d / "t.cpp"),
                    "-o", str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return {name: (int(per), int(pad)) for name, per, pad in (l.split() for l in out.splitlines())}


def test_a_whole_mi355x_takes_the_measured_shape(shapes):
    # B = 128 and B = 64 at 32 heads: 16 and 8 tiles per CU on 256 CUs
    assert shapes["full_b128"] == (512, 65536)
    assert shapes["full_b64"] == (256, 65536)
    # B = 48: 6 tiles per CU, the smallest large launch
    assert shapes["full_b48"] == (192, 65536)
    # 5 and 4 tiles per CU: neither choice
    assert shapes["full_b40"] == (0, 0)
    assert shapes["full_b32"] == (0, 0)
    # fp32 tiles are large from 12 per CU
    assert shapes["full_f32_b64"] == (0, 0)
    assert shapes["full_f32_b96"] == (384, 65536)
    # a tile count not divisible by 8 keeps dispatch order but takes the cap
    assert shapes["full_odd"] == (0, 65536)


def test_a_partitioned_or_unknown_device_gets_its_own_figures(shapes):
    # one XCD of 32 CUs: 16 tiles per CU is large, but the 8-XCD remap is off
    assert shapes["cpx_b16"] == (0, 65536)
    # the cap divides the device's own LDS per CU: 64 KiB / 2 - 8704 - 1024
    assert shapes["small_lds"] == (512, 64 * 1024 // 2 - 8704 - 1024)
    # nothing known: no large-launch choices
    assert shapes["unknown"] == (0, 0)


def test_overrides_win(shapes):
    # remap forced on a small launch; cap 3: 160 KiB / 3 - 8704 - 1024
    assert shapes["override_remap_cap3"] == (128, 160 * 1024 // 3 - 8704 - 1024)
    assert shapes["override_off"] == (0, 0)
