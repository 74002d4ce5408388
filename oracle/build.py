"""Build recipe for the oracle's C restatement: oracle/_build/liboracle.so.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Compiled with gcc at -O2
without -ffast-math, so the fp32 summation order in gemm_ref.c is the one the
source states.

The reference (willzeng274/kernel-rush-kawk) has no C/C++ sources for this
path (it is Python + Triton JIT), so there is no oracle/_ref build.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "gemm_ref.c"
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "liboracle.so"


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off",
           "-Wall", "-Wextra", str(SRC), "-lm", "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
