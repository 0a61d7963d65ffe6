"""Compile the C oracle (test infrastructure) into oracle/_build/liboracle.so.

The reference's kernels for this path are CUDA (.cu files built by nvcc with
ATen headers); nothing of them compiles here, so there is no oracle/_ref build.
The oracle is this repository's own C restatement, gdn_oracle.c.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "gdn_oracle.c"
OUT = HERE / "_build" / "liboracle.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off",
           "-fno-fast-math", "-Wall", str(SRC), "-o", str(tmp), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    tmp.replace(OUT)
    return OUT


if __name__ == "__main__":
    print(build())
