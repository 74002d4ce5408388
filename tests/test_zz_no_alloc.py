"""The allocation-free entry point, krk_gemm_bf16_noalloc, called through the
C ABI and compared bit for bit with krk_gemm_bf16 (its caller-workspace
counterpart, the same kernels and plan): two calls in a row on one stream,
the second with a smaller input, for split-K and unsplit plans; and the
error for a plan whose split-K partials do not fit the static scratch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from kernels import _lib
from kernels import gemm as G
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

NONE, SILU = _lib.EPILOGUE_NONE, _lib.EPILOGUE_SILU_MUL

# (name, epilogue, K, N, first M, second M): the second call is smaller.
PAIRS = [
    ("down, split K at both sizes", NONE, 9728, 2560, 64, 4),
    ("o, split K then unsplit", NONE, 4096, 2560, 32, 8),
    ("gate_up + SiLU*mul", SILU, 2560, 19456, 16, 3),
    ("qkv", NONE, 2560, 6144, 8, 1),
]


def say(*a):
    print("[case]", *a, flush=True)


def noalloc(x, w, y, epi):
    M, K = x.shape
    N = w.shape[0]
    rc = _lib.load().krk_gemm_bf16_noalloc(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(),
                                           y.stride(0), M, N, K, epi, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    return y


@pytest.mark.parametrize("name,epi,K,N,M1,M2", PAIRS, ids=[p[0] for p in PAIRS])
def test_noalloc_matches_workspace_entry_point(device, name, epi, K, N, M1, M2):
    w = R.randn_bf16((N, K), 9900 + N, 0.02).to(device)
    nout = N // 2 if epi == SILU else N
    for M in (M1, M2):
        say("noalloc", name, "M", M, G.plan(M, N, K, epi))
        x = R.randn_bf16((M, K), 9910 + M).to(device)
        want = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=device)
        nbytes = G.workspace_bytes(M, N, K, epi)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes else None
        G.gemm_into(x, w, want, epi, ws)
        got = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=device)
        noalloc(x, w, got, epi)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{name} M={M}: noalloc output differs from krk_gemm_bf16"
        ref = R.gateup_bf16(x.cpu(), w.cpu()) if epi == SILU else R.linear_bf16(x.cpu(), w.cpu())
        assert R.close(got.cpu(), ref).all(), f"{name} M={M}: outside 2e-2 + 1e-2|ref| of the oracle"


def test_noalloc_repeats_bit_exact(device):
    """The scratch keeps the last call's contents: the split-K counters must
    be back at zero after every call, so a repeat is bit-identical."""
    K, N = 9728, 2560
    w = R.randn_bf16((N, K), 9950, 0.02).to(device)
    x = R.randn_bf16((4, K), 9951).to(device)
    first = noalloc(x, w, torch.empty((4, N), dtype=torch.bfloat16, device=device), NONE).clone()
    for _ in range(3):
        again = noalloc(x, w, torch.full((4, N), float("nan"), dtype=torch.bfloat16, device=device), NONE)
        torch.cuda.synchronize()
        assert torch.equal(again, first)


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
