"""Build libkrk_gemm.so (the C-ABI GEMM library) and libkrk_probe.so (the
pure-read floor probe bench.py measures against) for gfx950 with hipcc.

Usage: ``python kernel-rush-kawk_amd/build_lib.py`` (or ``build()`` /
``build_probe()`` from Python).  The libraries are written next to this file
so they ship with the tree.  hipcc cross-compiles for gfx950 without a GPU
present.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
LIB = HERE / "libkrk_gemm.so"
SOURCES = [CSRC / "krk_gemm.hip"]
PROBE_LIB = HERE / "libkrk_probe.so"
PROBE_SOURCES = [CSRC / "krk_probe.hip"]
HEADERS = sorted(CSRC.glob("*.h")) + [ROOT / "include" / "krk_gemm.h"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU forms are kept out of the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def build(verbose: bool = False, extra_flags: list[str] | None = None, out: Path | None = None,
          sources: list[Path] | None = None) -> Path:
    """Compile the GEMM library (or ``sources`` into ``out``); always
    recompiles.  Returns the library path."""
    out = Path(out) if out else LIB
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, *(extra_flags or []), *map(str, sources or SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that
    # line is expected and not worth showing.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [l for l in (proc.stdout + proc.stderr).splitlines() if noise not in l]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, out)
    return out


def build_probe(verbose: bool = False) -> Path:
    """Compile libkrk_probe.so (bench.py's pure-read floor); always recompiles."""
    return build(verbose, out=PROBE_LIB, sources=PROBE_SOURCES)


if __name__ == "__main__":
    path = build(verbose=True)
    print(f"built {path}")
    print(f"built {build_probe(verbose=True)}")
    sys.exit(0)
