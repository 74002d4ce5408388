"""Every dispatch-table row at its real shape: the five Qwen3-4B projections
at every M from 1 to 64, plain and (qkv, gate_up, lm_head) normed, each run
on the plan the library picks for that M, against the CPU oracle.

Inputs are generated once per shape at M = 64 on the CPU (seeded) and the
oracle is computed once there; the call at M uses the first M rows of x, and
its output is compared with the first M rows of the M = 64 oracle (rows of a
projection are independent; the oracle's own fp32 summation order may differ
between M by one bf16 ulp, far inside the bar).  Bar: |y - ref| <= 2e-2 +
1e-2·|ref| everywhere; for normed calls xout = bf16(x + y) bit for bit.

This pins the planned geometry of every row — block counts, channels per
block, the ragged last round of a persistent grid, split counts, ring depths,
x held in registers or staged — at N = 2560 / 6144 / 19456 / 151936, which
the toy-shape sweeps of the kernel templates do not reach.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kernels import _lib
from kernels import gemm as G
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

NONE, SILU = _lib.EPILOGUE_NONE, _lib.EPILOGUE_SILU_MUL
# name -> (K, N_w, epilogue, normed)
SHAPES = {
    "qkv": (2560, 6144, NONE, True),
    "o": (4096, 2560, NONE, False),
    "gate_up": (2560, 19456, SILU, True),
    "down": (9728, 2560, NONE, False),
    "lm_head": (2560, 151936, NONE, True),
}
MS = list(range(1, 65))
EPS = 1e-6


def say(*a):
    print("[case]", *a, flush=True)


def _fail_detail(y, ref, ok, what):
    bad = np.argwhere(~ok)[:5]
    yf, rf = y.float().numpy(), ref.float().numpy()
    detail = ", ".join(f"{tuple(i)}: {yf[tuple(i)]} vs {rf[tuple(i)]}" for i in bad)
    return f"{what}: {(~ok).sum()} of {ok.size} outside 2e-2 + 1e-2|ref| ({detail})"


@pytest.fixture(scope="module")
def operands():
    """Per shape: CPU x[64, K], W, the residual branch d and gain, and the
    device copies; oracle outputs are computed lazily per shape."""
    cache = {}

    def get(name, device):
        if name not in cache:
            K, Nw, epi, normed = SHAPES[name]
            base = 6000 + 17 * list(SHAPES).index(name)
            x = R.randn_bf16((64, K), base + 1)
            w = R.randn_bf16((Nw, K), base + 2, 0.02)
            d = R.randn_bf16((64, K), base + 3, 0.5)
            wn = (R.randn_bf16((K,), base + 4, 0.1).float() + 1.0).to(torch.bfloat16)
            say("oracle", name, "M=64")
            ref = R.gateup_bf16(x, w) if epi == SILU else R.linear_bf16(x, w)
            nref = None
            if normed:
                fn = R.normed_gateup_bf16 if epi == SILU else R.normed_linear_bf16
                nref = fn(x, d, wn, EPS, w)
            cache[name] = dict(x=x, w=w, d=d, wn=wn, ref=ref, nref=nref, xd=x.to(device), wd=w.to(device),
                               dd=d.to(device), wnd=wn.to(device))
        return cache[name]

    return get


@pytest.mark.parametrize("name", list(SHAPES))
def test_every_row_of_the_plan(device, operands, name):
    K, Nw, epi, _ = SHAPES[name]
    op = operands(name, device)
    nout = Nw // 2 if epi == SILU else Nw
    seen = set()
    for M in MS:
        cfg = G.plan(M, Nw, K, epi)
        seen.add(tuple(sorted(cfg.items())))
        say(name, "M", M, cfg)
        y = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=device)
        nbytes = G.workspace_bytes(M, Nw, K, epi)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes else None
        G.gemm_into(op["xd"][:M], op["wd"], y, epi, ws)
        torch.cuda.synchronize()
        yc, ref = y.cpu(), op["ref"][:M]
        ok = R.close(yc, ref)
        assert ok.all(), _fail_detail(yc, ref, ok, f"{name} M={M} plan {cfg}")
    say(name, len(seen), "distinct plans over M = 1..64")


@pytest.mark.parametrize("name", [n for n, s in SHAPES.items() if s[3]])
def test_every_row_of_the_normed_plan(device, operands, name):
    K, Nw, epi, _ = SHAPES[name]
    op = operands(name, device)
    nout = Nw // 2 if epi == SILU else Nw
    ref_xout, ref = op["nref"]
    for M in MS:
        cfg = G.normed_plan(M, Nw, K, epi)
        say("normed", name, "M", M, cfg, "fused" if G.normed_fused(M, Nw, K, epi, cfg) else "prologue kernel")
        y = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=device)
        xout = torch.full((M, K), float("nan"), dtype=torch.bfloat16, device=device)
        nbytes = G.workspace_bytes(M, Nw, K, epi, normed=True)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes else None
        G.gemm_into(op["xd"][:M], op["wd"], y, epi, ws, norm=(op["dd"][:M], op["wnd"], xout, EPS))
        torch.cuda.synchronize()
        assert torch.equal(xout.cpu(), ref_xout[:M]), f"normed {name} M={M}: xout differs from bf16(x + y)"
        yc = y.cpu()
        ok = R.close(yc, ref[:M])
        assert ok.all(), _fail_detail(yc, ref[:M], ok, f"normed {name} M={M} plan {cfg}")
