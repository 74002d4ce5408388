"""Checks on the AMD assembly of the built library (our own code object).

The VALU kernel's LDS-staged paths issue the x (and branch) DMAs, then the
first chunk's weight loads, then wait with ``s_waitcnt vmcnt(N)`` for the
DMAs alone.  vmcnt retires in order, so the wait is right only if at least N
vector loads are issued after the last DMA and before the wait; a compiler
that moved a weight load below the wait (or above a DMA) would let a DMA
still be in flight when its LDS data is read.  This test disassembles every
``valu_gemm_kernel`` instantiation in libkrk_gemm.so and checks that bound.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "kernel-rush-kawk_amd" / "libkrk_gemm.so"
LLVM = Path("/opt/rocm/llvm/bin")
TOOLS = [LLVM / "llvm-objcopy", LLVM / "clang-offload-bundler", LLVM / "llvm-objdump"]


@pytest.fixture(scope="module")
def disassembly(tmp_path_factory):
    if not LIB.exists() or not all(t.exists() for t in TOOLS):
        pytest.skip("needs the built library and the ROCm LLVM tools")
    d = tmp_path_factory.mktemp("codeobj")
    fat, obj = d / "fatbin", d / "dev.o"
    subprocess.run([str(TOOLS[0]), f"--dump-section=.hip_fatbin={fat}", str(LIB)], check=True)
    subprocess.run([str(TOOLS[1]), "--unbundle", "--type=o", f"--input={fat}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={obj}"], check=True)
    out = subprocess.run([str(TOOLS[2]), "-d", "--mcpu=gfx950", "--no-show-raw-insn", str(obj)],
                         check=True, capture_output=True, text=True).stdout
    return out


def _functions(text: str):
    cur, body = None, []
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
        if m:
            if cur:
                yield cur, body
            cur, body = m.group(1), []
        elif cur:
            body.append(line.strip())
    if cur:
        yield cur, body


def test_valu_dma_waits_cover_only_the_dmas(disassembly):
    checked = 0
    for name, body in _functions(disassembly):
        if "valu_gemm_kernel" not in name:
            continue
        dmas = [i for i, l in enumerate(body) if l.startswith("global_load_lds")]
        if not dmas:
            continue
        loads, wait = 0, None
        for l in body[max(dmas) + 1:]:
            if l.startswith("global_load_dword"):
                loads += 1
            m = re.match(r"s_waitcnt\s.*vmcnt\((\d+)\)", l)
            if m:
                wait = int(m.group(1))
                break
        assert wait is not None, f"{name}: no vmcnt wait after the DMAs"
        assert wait <= loads, f"{name}: waits for vmcnt({wait}) with only {loads} loads issued after the last DMA"
        checked += 1
    assert checked >= 10, checked


def test_lds_x_in_registers_keeps_weight_stages_in_flight(disassembly):
    """The LDS-staged kernel's register-held-x variants (XPRE, the last
    template argument > 0) load x for the whole K, then the first weight
    stages, and the first stage waits only for what it stashes.  A full
    drain (vmcnt(0)) before the first barrier means the compiler sank an x
    load under a condition and waits for every weight stage there (seen
    once, 4-5% slower): no such wait may precede the first barrier."""
    checked = 0
    for name, body in _functions(disassembly):
        m = re.search(r"mfma_lds_kernelILi\d+ELi\d+ELi\d+ELi(\d+)ELb[01]ELb0ELb0ELi(\d+)EE", name)
        if not m or int(m.group(2)) == 0:
            continue
        first_barrier = next(i for i, l in enumerate(body) if l.startswith("s_barrier"))
        drains = [l for l in body[:first_barrier] if re.match(r"s_waitcnt\s.*vmcnt\(0\)", l)]
        assert not drains, f"{name}: {drains[0]} before the first barrier"
        checked += 1
    assert checked >= 16, checked
