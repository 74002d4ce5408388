"""The allocation-free entry point, krk_gemm_bf16_noalloc, called through the
C ABI and compared bit for bit with krk_gemm_bf16 (its caller-workspace
counterpart, the same kernels and plan).

* The first no-alloc call of the process is made under graph capture (the
  use the header advertises): the captured graph is replayed several times,
  with eager no-alloc calls of other shapes in between, and every replay must
  equal the eager krk_gemm_bf16 result.
* Two calls in a row on one stream, the second with a smaller input, on
  plans that split K (their counters and partials live in the shared static
  scratch) and on unsplit ones; the split-K cases assert that the plan
  really splits, so a dispatch-table change cannot drop the coverage.
* Repeats of a split-K call with a split-K call of another shape between
  them: every call must leave the shared counters at zero.
* The error for a plan whose split-K partials do not fit the static scratch.

The tests run in file order and share the process's scratch; the capture
test comes first on purpose.
"""

from __future__ import annotations

import pytest
import torch

from kernels import _lib
from kernels import gemm as G
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

NONE, SILU = _lib.EPILOGUE_NONE, _lib.EPILOGUE_SILU_MUL
# Projection shapes (K, N) of Qwen3-4B.
QKV, O, GATE_UP, DOWN = (2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560)


def say(*a):
    print("[case]", *a, flush=True)


def noalloc(x, w, y, epi):
    """krk_gemm_bf16_noalloc through ctypes on the current stream."""
    M, K = x.shape
    N = w.shape[0]
    rc = _lib.load().krk_gemm_bf16_noalloc(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(),
                                           y.stride(0), M, N, K, epi, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    return y


def with_workspace(x, w, epi):
    """The same projection through krk_gemm_bf16 with a fresh workspace."""
    M, K = x.shape
    N = w.shape[0]
    nout = N // 2 if epi == SILU else N
    y = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=x.device)
    nbytes = G.workspace_bytes(M, N, K, epi)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=x.device) if nbytes else None
    G.gemm_into(x, w, y, epi, ws)
    return y


def splits(M, shape, epi=NONE):
    K, N = shape
    return G.plan(M, N, K, epi)["splits"]


def operands(M, shape, seed, device):
    K, N = shape
    return R.randn_bf16((M, K), seed + M).to(device), R.randn_bf16((N, K), seed, 0.02).to(device)


def test_first_call_captured_in_a_graph(device):
    """down_proj at M = 64 splits K 3 ways; its first no-alloc call (the one
    that looks up the scratch and clears its counters) is recorded into a
    graph, and the graph is replayed five times, twice after eager no-alloc
    calls of other split-K shapes."""
    assert splits(64, DOWN) > 1
    x, w = operands(64, DOWN, 9800, device)
    want = with_workspace(x, w, NONE)
    torch.cuda.synchronize()
    got = torch.full_like(want, float("nan"))
    say("capture: first no-alloc call of the process, down M=64", G.plan(64, DOWN[1], DOWN[0]))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        noalloc(x, w, got, NONE)
    for rep in range(5):
        got.fill_(float("nan"))
        if rep in (2, 4):
            # eager split-K calls of other shapes on the same scratch
            xo, wo = operands(48, O, 9810, device)
            assert splits(48, O) > 1
            say("eager o M=48 between replays")
            eager = noalloc(xo, wo, torch.empty((48, O[1]), dtype=torch.bfloat16, device=device), NONE)
            assert torch.equal(eager, with_workspace(xo, wo, NONE))
            xd, wd = operands(24, DOWN, 9820, device)
            assert splits(24, DOWN) > 1
            say("eager down M=24 between replays")
            eager = noalloc(xd, wd, torch.empty((24, DOWN[1]), dtype=torch.bfloat16, device=device), NONE)
            assert torch.equal(eager, with_workspace(xd, wd, NONE))
        say("replay", rep)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}: the captured no-alloc call differs from krk_gemm_bf16"
    assert R.close(got.cpu(), R.linear_bf16(x.cpu(), w.cpu())).all()


# (name, epilogue, shape, first M, second M, whether both plans split K)
PAIRS = [
    ("down, split K at both sizes", NONE, DOWN, 64, 24, True),
    ("o, split K at both sizes", NONE, O, 64, 48, True),
    ("o, split K then unsplit", NONE, O, 48, 8, False),
    ("gate_up + SiLU*mul", SILU, GATE_UP, 16, 3, False),
    ("qkv", NONE, QKV, 8, 1, False),
]


@pytest.mark.parametrize("name,epi,shape,M1,M2,both_split", PAIRS, ids=[p[0] for p in PAIRS])
def test_noalloc_matches_workspace_entry_point(device, name, epi, shape, M1, M2, both_split):
    K, N = shape
    if both_split:
        assert splits(M1, shape, epi) > 1 and splits(M2, shape, epi) > 1, "the plan no longer splits K here"
    w = R.randn_bf16((N, K), 9900 + N, 0.02).to(device)
    nout = N // 2 if epi == SILU else N
    for M in (M1, M2):
        say("noalloc", name, "M", M, G.plan(M, N, K, epi))
        x = R.randn_bf16((M, K), 9910 + M).to(device)
        want = with_workspace(x, w, epi)
        got = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=device)
        noalloc(x, w, got, epi)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{name} M={M}: noalloc output differs from krk_gemm_bf16"
        ref = R.gateup_bf16(x.cpu(), w.cpu()) if epi == SILU else R.linear_bf16(x.cpu(), w.cpu())
        assert R.close(got.cpu(), ref).all(), f"{name} M={M}: outside 2e-2 + 1e-2|ref| of the oracle"


def test_split_k_repeats_bit_exact_through_the_python_wrapper(device):
    """The scratch keeps the last call's contents: every split-K call must
    leave the shared counters at zero, so down_proj at M = 24 (3 K splits)
    repeats bit-identically with a split-K o_proj call of another shape in
    between.  The calls go through kernels.gemm.gemm_noalloc."""
    assert splits(24, DOWN) > 1 and splits(64, O) > 1
    x, w = operands(24, DOWN, 9950, device)
    xo, wo = operands(64, O, 9960, device)
    want = with_workspace(x, w, NONE)
    want_o = with_workspace(xo, wo, NONE)
    for rep in range(4):
        say("repeat", rep)
        got = G.gemm_noalloc(x, w, torch.full_like(want, float("nan")))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"repeat {rep}: down M=24 differs"
        got_o = G.gemm_noalloc(xo, wo, torch.full_like(want_o, float("nan")))
        torch.cuda.synchronize()
        assert torch.equal(got_o, want_o), f"repeat {rep}: o M=64 differs"


def test_noalloc_rejects_plans_beyond_the_scratch(device):
    """M=8, N=65536, K=32768: the plan splits K 8 ways (the x slice must fit
    LDS), 16 MiB of partials against 4 MiB of scratch."""
    lib = _lib.load()
    x = torch.empty((8, 32768), dtype=torch.bfloat16, device=device)
    w = torch.empty((8, 32768), dtype=torch.bfloat16, device=device)  # never read: the call fails first
    y = torch.empty((8, 65536), dtype=torch.bfloat16, device=device)
    rc = lib.krk_gemm_bf16_noalloc(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(), y.stride(0),
                                   8, 65536, 32768, NONE, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.KRK_ERR_WORKSPACE
    assert "static scratch" in _lib.last_error()
