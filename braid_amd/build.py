"""Build libbraid_gdn.so (the C-ABI kernel library) for gfx950 with hipcc.

Run as ``python -m braid_amd.build``; ``__graft_entry__.build()`` calls
:func:`build`. The library lands in-tree at ``braid_amd/libbraid_gdn.so`` so it
travels with the source tree; nothing is installed.

Flags that matter for numerics:

* no fast-math: division and sqrt stay correctly rounded and ``expf`` /
  ``log1pf`` stay the accurate device-library routines, which is what torch's
  own elementwise kernels use (the in-kernel gates are compared bitwise
  against torch's spelling);
* ``-ffp-contract=off``: nothing is fused behind the source's back; every
  fused multiply-add in the kernels is an explicit ``fmaf``, so the
  decode and prefill kernels provably run the same operations;
* packed-fp32 instructions disabled (``-packed-fp32-ops``).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
ROOT = PKG.parent
LIB = PKG / "libbraid_gdn.so"
# The HBM stream probe bench.py measures the roofline ceiling with; not part
# of the drop-in ABI.
PROBE_LIB = PKG / "libbraid_probe.so"
PROBE_SOURCE = "hbm_probe.hip"
OBJ_DIR = PKG / "_build"

SOURCES = ["capi_common.cpp", "gdn_scan.hip", "conv1d_decode.hip", "quant_act.hip",
           "gated_norm.hip", "fp8_gemm.cpp", "fp8_gemm_stream.hip"]
# hipBLASLt for the FP8 GEMM. Its SONAME (libhipblaslt.so.1) matches the copy
# torch loads, so in a torch process the library binds to that one.
LIBS = ["-L/opt/rocm/lib", "-lhipblaslt"]

ARCH = os.environ.get("BRAID_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    return "hipcc"


def common_flags() -> list[str]:
    return [
        "-O3", "-std=c++17", "-fPIC",
        f"--offload-arch={ARCH}",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", str(ROOT / "include"),
        "-Wall", "-Wno-unused-result",
    ]


def _compile(src: str, defines: tuple = (), obj_dir: Path = OBJ_DIR) -> Path:
    obj_dir.mkdir(parents=True, exist_ok=True)
    out = obj_dir / (Path(src).stem + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [hipcc(), *common_flags(), *[f"-D{d}" for d in defines], *lang, "-c",
           str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    return out


def build(verbose: bool = False, defines: tuple = (), lib: Path = LIB) -> Path:
    """Compile every source and link the shared library. Always rebuilds.
    `defines` (NAME=VALUE strings) and `lib` select a tuning variant."""
    obj_dir = OBJ_DIR if lib == LIB else lib.parent / (lib.stem + "_obj")
    with ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, defines, obj_dir), SOURCES))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), *LIBS,
           "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    if lib == LIB:
        build_probe(verbose)
    return lib


def build_probe(verbose: bool = False) -> Path:
    """Compile and link libbraid_probe.so (the HBM stream probe)."""
    obj = _compile(PROBE_SOURCE)
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", str(obj), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {PROBE_LIB}")
    return PROBE_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
