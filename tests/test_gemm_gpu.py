"""GPU parity of the HIP skinny GEMM against the CPU oracle (north-star rule:
|y - ref| <= 2e-2 + 1e-2·|ref|, lm_head argmax bit-identical), plus the
stronger fp64 check: every output is a correct bf16 rounding of SOME fp32
summation of the exact products.

Inputs are generated on the CPU from seeded generators and copied, so the
oracle and the kernel see identical bits.  Every call goes through the C ABI
(kernels.gemm -> ctypes -> libkrk_gemm.so).
"""

from __future__ import annotations

import itertools
from pathlib import Path

import numpy as np
import pytest
import torch

from kernels import gemm as G
from kernels import _lib
from oracle import gemm_ref as R

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
NONE, SILU = _lib.EPILOGUE_NONE, _lib.EPILOGUE_SILU_MUL


def say(*a):
    print("[case]", *a, flush=True)


def krk(x, w, epilogue=NONE, config=None, device="cuda:0"):
    """Run the HIP GEMM on CPU bf16 inputs; return the CPU result."""
    xd, wd = x.to(device), w.to(device)
    M, N = x.shape[0], w.shape[0]
    nout = N // 2 if epilogue == SILU else N
    # NaN-filled, so an output the kernel fails to write cannot pass by
    # holding a previous call's correct result (torch's allocator reuses blocks)
    y = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=device)
    nbytes = G.workspace_bytes(M, N, x.shape[1], epilogue, config)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes else None
    G.gemm_into(xd, wd, y, epilogue, ws, config)
    torch.cuda.synchronize()
    return y.cpu()


def assert_parity(y, ref, what):
    ok = R.close(y, ref)
    if not ok.all():
        bad = np.argwhere(~ok)[:5]
        yf, rf = y.float().numpy(), ref.float().numpy()
        detail = ", ".join(f"{tuple(i)}: {yf[tuple(i)]} vs {rf[tuple(i)]}" for i in bad)
        pytest.fail(f"{what}: {(~ok).sum()} of {ok.size} outside 2e-2 + 1e-2|ref| ({detail})")


def assert_fp32_rounding(y, x, w, what):
    exact, mag = R.linear_exact(x, w)
    ok = R.within_fp32_bound(y, exact, mag, x.shape[1])
    assert ok.all(), f"{what}: {(~ok).sum()} outputs are not a rounding of any fp32 sum"


def check_linear(x, w, what, config=None):
    say(what, tuple(x.shape), tuple(w.shape), config)
    y = krk(x, w, NONE, config)
    assert_parity(y, R.linear_bf16(x, w), what)
    assert_fp32_rounding(y, x, w, what)
    return y


def check_gateup(x, w, what, config=None):
    say(what, tuple(x.shape), tuple(w.shape), config)
    y = krk(x, w, SILU, config)
    assert_parity(y, R.gateup_bf16(x, w), what)
    return y


# ---------------------------------------------------------------- fixtures


LIN = np.load(GOLDEN / "linear_cases.npz")
GU = np.load(GOLDEN / "gateup_cases.npz")


@pytest.mark.parametrize("name", sorted({k.split("/")[0] for k in LIN.files}))
def test_golden_linear(device, name):
    x, w, y = (R.from_bits(LIN[f"{name}/{k}"]) for k in ("x", "w", "y"))
    got = check_linear(x, w, f"golden {name}")
    assert_parity(got, y, f"golden {name} vs fixture")


@pytest.mark.parametrize("name", sorted({k.split("/")[0] for k in GU.files}))
def test_golden_gateup(device, name):
    x, w, y = (R.from_bits(GU[f"{name}/{k}"]) for k in ("x", "w", "y"))
    got = check_gateup(x, w, f"golden {name}")
    assert_parity(got, y, f"golden {name} vs fixture")


# ---------------------------------------------------------------- BASELINE configs


def test_c1_qkv_m1(device):
    x = R.randn_bf16((1, 2560), R.seed_for(1, 0, "x"))
    w = R.randn_bf16((6144, 2560), R.seed_for(1, 0, "qkv"), 0.02)
    check_linear(x, w, "C1 qkv M=1")


@pytest.mark.parametrize("M", [1, 4])
def test_c2_down_splitk(device, M):
    x = R.randn_bf16((M, 9728), R.seed_for(2, 0, "x"), 0.5)
    w = R.randn_bf16((2560, 9728), R.seed_for(2, 0, "down"), 0.02)
    check_linear(x, w, f"C2 down M={M}")


def test_c3_gateup_m8(device):
    x = R.randn_bf16((8, 2560), R.seed_for(3, 0, "x"))
    w = R.randn_bf16((19456, 2560), R.seed_for(3, 0, "gate_up"), 0.02)
    check_gateup(x, w, "C3 gate_up+silu M=8")


def _lm_argmax_check(x, lm, what, device):
    say(what, tuple(x.shape))
    logits = krk(x, lm)
    ref = R.linear_bf16(x, lm)
    assert_parity(logits, ref, what)
    got, want = R.argmax_rows(logits), R.argmax_rows(ref)
    if not torch.equal(got, want):
        rows = (got != want).nonzero().flatten().tolist()
        info = [(r, want[r].item(), got[r].item(), ref[r, want[r]].item(), ref[r, got[r]].item()) for r in rows[:4]]
        pytest.fail(f"{what}: argmax differs on rows {rows} (row, want, got, ref[want], ref[got]): {info}")
    # the device-side argmax of the device logits agrees too
    assert torch.equal(torch.argmax(logits.to(device), dim=-1).cpu(), want)


@pytest.mark.parametrize("shape", ["qkv", "o", "gate_up", "down"])
def test_c5_verify_m64(device, shape):
    K, N, epi = R.SHAPES[shape]
    x = R.randn_bf16((64, K), R.seed_for(5, 0, "x") + K)
    w = R.randn_bf16((N, K), R.seed_for(5, 0, shape), 0.02)
    if epi == "silu_mul":
        check_gateup(x, w, f"C5 {shape} M=64")
    else:
        check_linear(x, w, f"C5 {shape} M=64")


@pytest.fixture(scope="module")
def lm_head():
    return R.randn_bf16((R.VOCAB, R.HIDDEN), R.seed_for(4, 99, "lm_head"), 0.02)


@pytest.mark.parametrize("M", [64, 32, 8, 1])
def test_lm_head_argmax(device, lm_head, M):
    x = R.randn_bf16((M, R.HIDDEN), R.seed_for(5, M, "x"))
    _lm_argmax_check(x, lm_head, f"lm_head M={M}", device)


@pytest.mark.parametrize("layer", range(R.LAYERS))
def test_c4_sweep_layers_m32(device, layer):
    """C4: M=32 through every layer's four projections, each layer with its
    own seeded weights (teacher-forced: each GEMM is fed the oracle's input,
    so bf16 differences do not compound).  Layers 0, 17 and 35 also get the
    fp64 rounding check."""
    M = 32
    check = check_linear if layer in (0, 17, 35) else _check_linear_parity
    h = R.randn_bf16((M, R.HIDDEN), R.seed_for(4, layer, "x"))
    wqkv = R.randn_bf16((6144, R.HIDDEN), R.seed_for(4, layer, "qkv"), 0.02)
    wo = R.randn_bf16((R.HIDDEN, R.Q_WIDTH), R.seed_for(4, layer, "o"), 0.02)
    wgu = R.randn_bf16((2 * R.INTER, R.HIDDEN), R.seed_for(4, layer, "gate_up"), 0.02)
    wd = R.randn_bf16((R.HIDDEN, R.INTER), R.seed_for(4, layer, "down"), 0.02)
    qkv = check(h, wqkv, f"C4 L{layer} qkv")
    attn = R.linear_bf16(h, wqkv)[:, :R.Q_WIDTH].contiguous()  # stand-in attention output
    check(attn, wo, f"C4 L{layer} o")
    act = check_gateup(h, wgu, f"C4 L{layer} gate_up")
    check(R.gateup_bf16(h, wgu), wd, f"C4 L{layer} down")
    assert qkv.shape == (M, 6144) and act.shape == (M, R.INTER)


def _check_linear_parity(x, w, what, config=None):
    say(what, tuple(x.shape), tuple(w.shape), config)
    y = krk(x, w, NONE, config)
    assert_parity(y, R.linear_bf16(x, w), what)
    return y


# ---------------------------------------------------------------- edge cases


def test_every_m_from_1_to_64(device):
    K, N = 4096, 160
    w = R.randn_bf16((N, K), 7001, 0.02)
    xs = R.randn_bf16((64, K), 7002)
    for M in range(1, 65):
        check_linear(xs[:M].contiguous(), w, f"M sweep M={M}")


@pytest.mark.parametrize("M", [65, 100, 130])
def test_rows_beyond_64_are_chunked(device, M):
    x = R.randn_bf16((M, 2560), 7100 + M)
    w = R.randn_bf16((96, 2560), 7200, 0.02)
    check_linear(x, w, f"chunked M={M}")
    wgu = R.randn_bf16((64, 2560), 7300, 0.02)
    check_gateup(x, wgu, f"chunked gateup M={M}")


@pytest.mark.parametrize("M,N,K", [(1, 17, 40), (3, 100, 136), (5, 1, 8), (16, 33, 2568), (40, 250, 520),
                                   (64, 18, 9736), (7, 2560, 24)])
def test_ragged_shapes(device, M, N, K):
    x = R.randn_bf16((M, K), 7400 + M + N)
    w = R.randn_bf16((N, K), 7500 + K, 0.02)
    check_linear(x, w, f"ragged M={M} N={N} K={K}")


@pytest.mark.parametrize("M,I,K", [(1, 24, 2560), (8, 40, 136), (64, 8, 264), (33, 100, 1000)])
def test_ragged_gateup(device, M, I, K):
    x = R.randn_bf16((M, K), 7600 + M)
    w = R.randn_bf16((2 * I, K), 7700 + I, 0.02)
    check_gateup(x, w, f"ragged gateup M={M} I={I} K={K}")


# One GPU's shard of each projection under 8-way tensor parallelism (the
# narrow-N / short-K shapes a multi-GPU deployment would run per GPU): QKV and
# lm_head column-parallel, gate_up with gate and up rows sharded together, o
# and down row-parallel.
TP8_SHARDS = {"qkv": (768, 2560, NONE), "gate_up": (2 * 1216, 2560, SILU), "o": (2560, 512, NONE),
              "down": (2560, 1216, NONE), "lm_head": (18992, 2560, NONE)}


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 13, 16, 24, 32, 48, 64])
@pytest.mark.parametrize("shard", sorted(TP8_SHARDS))
def test_tp8_shard_shapes(device, shard, M):
    N, K, epi = TP8_SHARDS[shard]
    x = R.randn_bf16((M, K), 7800 + M + K)
    w = R.randn_bf16((N, K), 7900 + N, 0.02)
    say("tp8 shard", shard, M, G.plan(M, N, K, epi))
    if epi == SILU:
        check_gateup(x, w, f"tp8 {shard} M={M}")
    elif shard == "lm_head":
        _lm_argmax_check(x, w, f"tp8 lm_head M={M}", device)
    else:
        check_linear(x, w, f"tp8 {shard} M={M}")


def test_strided_operands(device):
    """x a column slice of a wider buffer (ldx > K), y written into a wider buffer."""
    K, N, M = 2560, 300, 5
    big = R.randn_bf16((M, K + 64), 7800)
    w = R.randn_bf16((N, K), 7801, 0.02)
    say("strided", M, N, K)
    xd = big.to(device)[:, 32:32 + K]
    assert xd.stride(0) == K + 64
    ybig = torch.full((M, N + 24), 7.0, dtype=torch.bfloat16, device=device)
    nbytes = G.workspace_bytes(M, N, K)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes else None
    G.gemm_into(xd, w.to(device), ybig[:, 8:8 + N], NONE, ws)
    torch.cuda.synchronize()
    got = ybig.cpu()
    assert_parity(got[:, 8:8 + N], R.linear_bf16(big[:, 32:32 + K], w), "strided")
    assert (got[:, :8].float() == 7.0).all() and (got[:, 8 + N:].float() == 7.0).all(), "wrote outside y"


def test_special_inputs_exact(device):
    """x = 0 gives 0; a one-hot row reproduces one column of W^T bit-exactly
    (a single product is exact), which pins the (m, n, k) indexing."""
    K, N = 4096, 2560
    w = R.randn_bf16((N, K), 7900, 0.02)
    assert (krk(torch.zeros(3, K, dtype=torch.bfloat16), w).float() == 0).all()
    cols = [0, 1, 31, 32, 511, 2047, K - 1]
    oh = torch.zeros(len(cols), K, dtype=torch.bfloat16)
    for r, c in enumerate(cols):
        oh[r, c] = 1.0
    say("one-hot", cols)
    y = krk(oh, w)
    for r, c in enumerate(cols):
        assert torch.equal(y[r], w[:, c]), f"one-hot row {r} (k={c}) wrong"
    y2 = krk(-oh, w)
    assert torch.equal(y2, -y)


# One configuration of every kernel family, with and without split K.
SPECIAL_FAMILIES = [
    ("valu", 4, dict(kernel=_lib.KERNEL_VALU, splits=1)),
    ("valu split-K", 3, dict(kernel=_lib.KERNEL_VALU, splits=3)),
    ("valu x in registers", 2, dict(kernel=_lib.KERNEL_VALU, splits=2)),
    ("lds-staged", 16, dict(kernel=_lib.KERNEL_MFMA_LDS, splits=1)),
    ("lds-staged split-K", 24, dict(kernel=_lib.KERNEL_MFMA_LDS, splits=3)),
    ("lds-staged 24 channels split-K", 20, dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=4, channels=24, splits=2)),
    ("lds-staged x in registers", 20, dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=2, k_chunk=512, splits=1, x_preload=2)),
    ("stream", 33, dict(kernel=_lib.KERNEL_STREAM, splits=1)),
    ("stream split-K", 8, dict(kernel=_lib.KERNEL_STREAM, splits=2)),
    ("register mfma split-K", 13, dict(kernel=_lib.KERNEL_MFMA, splits=2)),
    ("wave-sliced", 8, dict(kernel=_lib.KERNEL_SLICE, channels=10, splits=1)),
    ("wave-sliced 128-k chunks", 12, dict(kernel=_lib.KERNEL_SLICE, k_chunk=128, channels=13, splits=1)),
    ("wave-sliced split-K", 20, dict(kernel=_lib.KERNEL_SLICE, channels=24, splits=3)),
]
# The wave-sliced kernel computes plain projections only.
SPECIAL_CASES = [(f, M, c, epi) for f, M, c in SPECIAL_FAMILIES for epi in (NONE, SILU)
                 if not (epi == SILU and c["kernel"] == _lib.KERNEL_SLICE)]


# (a, b) pairs whose fp32 sum a + b is exact and lies exactly halfway between
# two bf16 values (or just above it): the epilogue's round-to-nearest-even
# decides the output bits.
TIE_PAIRS = [(1.0, 2.0 ** -8), (1.0 + 2.0 ** -7, 2.0 ** -8), (1.0, 2.0 ** -8 + 2.0 ** -15), (256.0, 1.0),
             (258.0, 1.0), (-1.0, -(2.0 ** -8)), (-(1.0 + 2.0 ** -7), -(2.0 ** -8)), (3.0, 2.0 ** -7),
             (2.0 ** -120, 2.0 ** -128), (65280.0, 128.0)]


@pytest.mark.parametrize("family,M,config", SPECIAL_FAMILIES, ids=[f[0] for f in SPECIAL_FAMILIES])
def test_round_half_even_outputs(device, family, M, config):
    """Each row of x holds two ones (in different halves of K, so different
    splits and stages); each W channel holds a tie pair (a, b) at those two
    columns.  y = bf16(a + b) with the sum exact in fp32, so the output bits
    are fixed by round-to-nearest-even alone, in every kernel family."""
    K, N = 2560, 96
    w = R.randn_bf16((N, K), 7950, 0.02)
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    a = torch.tensor([TIE_PAIRS[n % len(TIE_PAIRS)][0] for n in range(N)], dtype=torch.bfloat16)
    b = torch.tensor([TIE_PAIRS[n % len(TIE_PAIRS)][1] for n in range(N)], dtype=torch.bfloat16)
    assert torch.equal(a.float(), torch.tensor([p[0] for p in TIE_PAIRS] * 10)[:N]) and \
        torch.equal(b.float(), torch.tensor([p[1] for p in TIE_PAIRS] * 10)[:N]), "tie pairs must be bf16 values"
    for m in range(M):
        k1 = (37 + 71 * m) % (K // 2)
        k2 = K // 2 + (5 + 53 * m) % (K // 2)
        x[m, k1] = 1.0
        x[m, k2] = 1.0
        w[:, k1] = a
        w[:, k2] = b
    expected = (a.float() + b.float()).to(torch.bfloat16).expand(M, N)
    say("round half even", family, M, config)
    y = krk(x, w, NONE, config)
    assert torch.equal(y.view(torch.int16), expected.view(torch.int16)), \
        f"{family}: {(y != expected).sum().item()} outputs off the round-to-nearest-even bits"


def _special_operands(M, N, K, seed):
    """Random operands with NaN, +-inf and -0 planted in x rows and W rows.
    x: row 0 NaN at one k; row 1 +inf; row 2 -inf and +inf (products of
    either sign: NaN or an infinity per channel); row 3 all -0.  W: channel 3
    NaN; channel 5 +inf; channel 6 -inf; channel 9 all -0; channel 10 +inf at
    the k where x row 1 is +inf."""
    x = R.randn_bf16((M, K), seed)
    w = R.randn_bf16((N, K), seed + 1, 0.02)
    inf, nan = float("inf"), float("nan")
    x[0, 5] = nan
    x[min(1, M - 1), 17] = inf
    if M > 2:
        x[2, K // 3] = -inf
        x[2, K - 1] = inf
    if M > 3:
        x[3, :] = -0.0
    w[3, 7] = nan
    w[5, K // 2] = inf
    w[6, 1] = -inf
    w[9, :] = -0.0
    w[10, 17] = inf
    return x, w


def _assert_special_parity(y, ref, what):
    """NaN exactly where the oracle has NaN, infinities equal (with sign),
    every finite value within the north-star tolerance.  (The sign of a zero
    result depends on the summation order and is not compared: -0 == +0.)"""
    nan_y, nan_r = y.float().isnan(), ref.float().isnan()
    assert torch.equal(nan_y, nan_r), f"{what}: NaN mask differs at {(nan_y != nan_r).nonzero()[:6].tolist()}"
    inf_r = ref.float().isinf()
    assert torch.equal(y.float().isinf(), inf_r), f"{what}: infinity mask differs"
    assert torch.equal(y.float()[inf_r], ref.float()[inf_r]), f"{what}: infinity signs differ"
    fin = ~(nan_r | inf_r)
    yf, rf = y.float()[fin], ref.float()[fin]
    bad = (yf - rf).abs() > 2e-2 + 1e-2 * rf.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} finite values outside 2e-2 + 1e-2|ref|"


@pytest.mark.parametrize("family,M,config,epi", SPECIAL_CASES,
                         ids=[f"{c[0]}-{'plain' if c[3] == NONE else 'silu_mul'}" for c in SPECIAL_CASES])
def test_special_values_propagate(device, family, M, config, epi):
    """NaN, +-inf and -0 in x and in W rows, through every kernel family
    (VALU dot2, LDS-staged MFMA, stream MFMA, register MFMA), the split-K
    fix-up and the SiLU*mul epilogue (expf at +-inf), against F.linear /
    swiglu on the CPU."""
    K = 2048
    N = 64 if epi == NONE else 96
    x, w = _special_operands(M, N, K, 9100 + M)
    if epi == SILU:
        # gate rows 0..47, up rows 48..95: put specials in gate and up rows
        w[48 + 3, 11] = float("nan")   # up row of channel 3 (gate row 3 is NaN too)
        w[48 + 20, 17] = -float("inf")  # up row of channel 20: x row 1 gives -inf * +inf
        w[30, 17] = -float("inf")      # gate row of channel 30 at x row 1's +inf: silu(-inf)
    cfg = dict(config)
    say("special values", family, "M", M, "epi", epi, cfg)
    y = krk(x, w, epi, cfg)
    ref = R.gateup_bf16(x, w) if epi == SILU else R.linear_bf16(x, w)
    # the planted values do reach the outputs
    assert ref.float().isnan().any() and ref.float().isinf().any()
    _assert_special_parity(y, ref, f"{family} {'silu' if epi == SILU else 'plain'}")
    if epi == NONE and M > 3:
        # rows from 3 on hold no NaN or infinity (row 3 is all -0)
        assert (y[3:, 9].float() == 0).all(), "a -0 weight row gives zeros"
        assert (y[3].float().nan_to_num(1.0) == 0).sum() == N - 4, "a -0 x row gives zeros (NaN at the 4 NaN/inf channels)"


# ---------------------------------------------------------------- configurations


def test_deterministic_repeat(device):
    x = R.randn_bf16((4, 9728), 8000, 0.5)
    w = R.randn_bf16((2560, 9728), 8001, 0.02)
    say("determinism", G.plan(4, 2560, 9728))
    a = krk(x, w)
    for _ in range(3):
        assert torch.equal(krk(x, w), a)


def _mfma_configs(M, silu):
    mt_min = -(-min(M, 64) // 16)
    for mt, nt, u, wv, sp in itertools.product(range(mt_min, 5), (1, 2, 4), (2, 4, 8), (1, 2, 4), (1, 2, 3, 8)):
        if silu and nt % 2:
            continue
        if mt * nt * u > 32:  # large register footprints spill; not worth a slot here
            continue
        if wv * mt * nt >= 64:  # reduction area past the 64 KB LDS budget: rejected by the host
            continue
        yield dict(kernel=_lib.KERNEL_MFMA, m_tiles=mt, n_tiles=nt, unroll=u, waves=wv, splits=sp)


@pytest.mark.parametrize("M", [1, 13, 64])
def test_all_mfma_configs_agree(device, M):
    """Every configuration computes the same function: each is a correct
    rounding of an fp32 order and within tolerance of the oracle."""
    K, N = 1024, 96
    x = R.randn_bf16((M, K), 8100 + M)
    w = R.randn_bf16((N, K), 8101, 0.02)
    ref = R.linear_bf16(x, w)
    exact, mag = R.linear_exact(x, w)
    for cfg in _mfma_configs(M, False):
        say("config", M, cfg)
        y = krk(x, w, NONE, cfg)
        assert_parity(y, ref, f"config {cfg}")
        assert R.within_fp32_bound(y, exact, mag, K).all(), f"config {cfg}"


def test_all_mfma_gateup_configs_agree(device):
    M, K, I = 8, 512, 40
    x = R.randn_bf16((M, K), 8200)
    w = R.randn_bf16((2 * I, K), 8201, 0.02)
    ref = R.gateup_bf16(x, w)
    for cfg in _mfma_configs(M, True):
        say("gateup config", cfg)
        assert_parity(krk(x, w, SILU, cfg), ref, f"gateup config {cfg}")


def _lds_configs(M, silu):
    mt_min = -(-min(M, 64) // 16)
    for mt, nt, pf, kc, sp in itertools.product(range(mt_min, 5), (1, 2, 4), (2, 3), (256, 512), (1, 2, 3, 9)):
        if silu and nt % 2:
            continue
        yield dict(kernel=_lib.KERNEL_MFMA_LDS, m_tiles=mt, n_tiles=nt, unroll=pf, k_chunk=kc, splits=sp)


def _stream_configs(M, K):
    mt_min = -(-min(M, 64) // 16)
    for mt, sp, d in itertools.product(range(mt_min, 5), (1, 2, 3), (2, 3, 5, 8)):
        yield dict(kernel=_lib.KERNEL_STREAM, m_tiles=mt, splits=sp, unroll=d)


def _valu_configs(silu, depths=(2, 3, 5, 7, 19)):
    for wv, nt, d, sp in itertools.product((1, 5, 8), (1, 2, 4), depths, (1, 3)):
        if silu and nt % 2:
            continue
        yield dict(kernel=_lib.KERNEL_VALU, waves=wv, n_tiles=nt, unroll=d, splits=sp)


def _run_configs(x, w, epi, configs):
    """Run every configuration the library accepts; check each against the oracle."""
    ref = R.gateup_bf16(x, w) if epi == SILU else R.linear_bf16(x, w)
    bound = None if epi == SILU else R.linear_exact(x, w)
    ran = 0
    for cfg in configs:
        if G.workspace_bytes(x.shape[0], w.shape[0], x.shape[1], epi, cfg) == 0 and cfg.get("splits", 1) > 1:
            continue  # rejected configuration (e.g. x-register budget)
        say("config", tuple(x.shape), tuple(w.shape), epi, cfg)
        try:
            y = krk(x, w, epi, cfg)
        except ValueError as e:
            if "krk error -6" in str(e):
                continue
            raise
        assert_parity(y, ref, f"config {cfg}")
        if bound is not None:
            assert R.within_fp32_bound(y, bound[0], bound[1], x.shape[1]).all(), f"config {cfg}"
        ran += 1
    assert ran > 0


@pytest.mark.parametrize("M,N,K", [(1, 96, 1536), (13, 200, 1000), (40, 96, 2568), (64, 130, 520)])
def test_all_lds_configs_agree(device, M, N, K):
    x = R.randn_bf16((M, K), 8700 + M)
    w = R.randn_bf16((N, K), 8701 + N, 0.02)
    _run_configs(x, w, NONE, _lds_configs(M, False))


def _lds_channel_configs(M, silu):
    """LDS-staged configurations whose blocks hold fewer channels than their
    tiles: every multiple of 8 below the tiles' width."""
    mt_min = -(-min(M, 64) // 16)
    for mt, nt, sp in itertools.product(range(mt_min, 5), (1, 2, 4), (1, 3)):
        if silu and nt % 2:
            continue
        full = 16 * (nt // 2 if silu else nt)
        for ch in range(8, full, 8):
            yield dict(kernel=_lib.KERNEL_MFMA_LDS, m_tiles=mt, n_tiles=nt, unroll=2, k_chunk=256, splits=sp,
                       channels=ch)


@pytest.mark.parametrize("M,N,K,epi", [(1, 96, 1536, NONE), (13, 200, 1000, NONE), (40, 6144, 2560, NONE),
                                       (64, 130, 520, NONE), (5, 2 * 96, 2560, SILU), (24, 2 * 200, 1032, SILU)])
def test_lds_partial_channel_configs(device, M, N, K, epi):
    """Blocks of fewer channels than their tiles (the rest padding, neither
    loaded nor stored) give the oracle's results, with and without split K,
    at N that is and is not a multiple of the channel count."""
    x = R.randn_bf16((M, K), 8750 + M)
    w = R.randn_bf16((N, K), 8751 + N, 0.02)
    _run_configs(x, w, epi, _lds_channel_configs(M, epi == SILU))


def _lds_xpre_configs(M, silu):
    """LDS-staged configurations that hold x in registers for the whole K
    (x_preload = 2): one or two x tiles, one or two weight tiles, two or
    three stages in flight, all of the tiles' channels and 8 fewer."""
    mt_min = -(-min(M, 64) // 16)
    for mt, nt, pf in itertools.product(range(mt_min, 3), (1, 2), (2, 3)):
        if silu and nt % 2:
            continue
        full = 16 * (nt // 2 if silu else nt)
        for ch in sorted({full, max(8, full - 8)}):
            yield dict(kernel=_lib.KERNEL_MFMA_LDS, m_tiles=mt, n_tiles=nt, unroll=pf, k_chunk=512, splits=1,
                       channels=ch, x_preload=2)


@pytest.mark.parametrize("M,N,K,epi", [(1, 96, 1536, NONE), (9, 200, 1000, NONE), (16, 6144, 2560, NONE),
                                       (24, 520, 2056, NONE), (32, 130, 512, NONE), (3, 96, 8, NONE),
                                       (13, 2 * 96, 2560, SILU), (20, 2 * 200, 1032, SILU), (32, 2 * 600, 2048, SILU),
                                       (16, 2560, 4096, NONE), (32, 2560, 4096, NONE), (9, 200, 2568, NONE),
                                       (24, 520, 3584, NONE), (32, 2 * 300, 4096, SILU), (5, 96, 4088, NONE),
                                       (9, 2560, 9728, NONE), (16, 200, 9000, NONE), (12, 96, 4616, NONE),
                                       (1, 130, 9720, NONE)])
def test_lds_x_in_registers_configs(device, M, N, K, epi):
    """x held in registers for the whole K (one to nineteen 512-k stages: the
    5-stage variant up to K = 2560, the 8-stage one up to 4096 and, with one
    x tile and one weight tile, the 19-stage one above, each running the
    stages past K as zeros; ragged K down to a single 8-element chunk, ragged
    N, partial channel blocks, both epilogues) gives the oracle's results,
    within the fp32 bound."""
    x = R.randn_bf16((M, K), 8780 + M)
    w = R.randn_bf16((N, K), 8781 + N, 0.02)
    _run_configs(x, w, epi, _lds_xpre_configs(M, epi == SILU))


@pytest.mark.parametrize("kernel", [_lib.KERNEL_MFMA, _lib.KERNEL_MFMA_LDS, _lib.KERNEL_VALU, _lib.KERNEL_SLICE])
@pytest.mark.parametrize("splits", [8, 9, 16, 17, 32])
def test_many_splits_fixed_order(device, kernel, splits):
    """Split counts around and past the fix-up's load batch (8 splits per round
    trip): the combined result is still a correct fp32 rounding, and equal
    for repeated calls."""
    M, N, K = (5, 96, 32768) if kernel == _lib.KERNEL_VALU else (20, 96, 32768)
    x = R.randn_bf16((M, K), 9100 + splits)
    w = R.randn_bf16((N, K), 9101, 0.02)
    cfg = dict(kernel=kernel, splits=splits)
    say("many splits", kernel, splits, M, N, K)
    y = krk(x, w, NONE, cfg)
    assert_parity(y, R.linear_bf16(x, w), f"config {cfg}")
    exact, mag = R.linear_exact(x, w)
    assert R.within_fp32_bound(y, exact, mag, K).all(), f"config {cfg}"
    assert torch.equal(y, krk(x, w, NONE, cfg))


@pytest.mark.parametrize("M,N,K", [(1, 96, 1536), (13, 200, 1000), (40, 96, 2568), (64, 130, 520), (5, 4099, 2048)])
def test_all_stream_configs_agree(device, M, N, K):
    x = R.randn_bf16((M, K), 8800 + M)
    w = R.randn_bf16((N, K), 8801 + N, 0.02)
    _run_configs(x, w, NONE, _stream_configs(M, K))


def _slice_configs(M):
    """Wave-sliced configurations: 64- and 128-k chunks, 2 or 3 in flight,
    channel counts from one to two full tiles (partial 8- and 4-row groups),
    K unsplit and split (more splits than some waves have chunks)."""
    for kc, d, ch, sp in itertools.product((64, 128), (2, 3), (1, 5, 8, 10, 13, 16, 17, 24, 32), (1, 2, 7)):
        yield dict(kernel=_lib.KERNEL_SLICE, k_chunk=kc, unroll=d, channels=ch, splits=sp)


@pytest.mark.parametrize("M,N,K", [(1, 96, 1536), (5, 200, 1000), (8, 2560, 4096), (13, 33, 2568), (16, 130, 8),
                                   (24, 6144, 520), (32, 97, 1096), (9, 2560, 9728)])
def test_all_slice_configs_agree(device, M, N, K):
    """The wave-sliced kernel under every instantiated variant: ragged K (a
    tail chunk with its pieces past K masked, and K below one chunk), N that
    is not a multiple of the block's channels (its last block loads clamped
    rows it does not store), M that leaves a partial x group, and split K,
    against the oracle and within the fp32 bound."""
    x = R.randn_bf16((M, K), 8850 + M)
    w = R.randn_bf16((N, K), 8851 + N, 0.02)
    _run_configs(x, w, NONE, _slice_configs(M))


@pytest.mark.parametrize("M,I,K", [(1, 40, 1536), (8, 52, 1000), (33, 24, 2568), (64, 100, 520)])
def test_gateup_configs_all_kernels(device, M, I, K):
    x = R.randn_bf16((M, K), 8900 + M)
    w = R.randn_bf16((2 * I, K), 8901 + I, 0.02)
    _run_configs(x, w, SILU, itertools.chain(_lds_configs(M, True), _stream_configs(M, K)))


@pytest.mark.parametrize("M,N,K", [(1, 96, 1536), (3, 200, 1000), (8, 130, 2568), (5, 4099, 520), (2, 40, 8),
                                   (7, 33, 4096)])
def test_all_valu_configs_agree(device, M, N, K):
    """Row-streaming VALU kernel: every (waves, rows per wave, blocks in flight,
    splits) choice, with a ragged last K block (lanes past K masked), K below
    one block, and channel counts that leave a workgroup partly empty."""
    x = R.randn_bf16((M, K), 9100 + M)
    w = R.randn_bf16((N, K), 9101 + N, 0.02)
    _run_configs(x, w, NONE, _valu_configs(False))


@pytest.mark.parametrize("M,I,K", [(1, 40, 1536), (8, 52, 1000), (4, 9, 2568)])
def test_valu_gateup_configs(device, M, I, K):
    x = R.randn_bf16((M, K), 9200 + M)
    w = R.randn_bf16((2 * I, K), 9201 + I, 0.02)
    _run_configs(x, w, SILU, _valu_configs(True))


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_valu_qwen_shapes(device, M):
    """The VALU kernel on the real projection shapes, including down's 19
    K blocks (several passes of the block loop), the widest split and
    workgroups of 3, 5 and 6 waves (grids whose last workgroup is partly
    past N: o's 2560 channels over 3 x 1 per workgroup, qkv's 6144 over
    5 x 2)."""
    for name, (N, K, epi) in {"qkv": (6144, 2560, NONE), "o": (2560, 4096, NONE), "down": (2560, 9728, NONE),
                              "gate_up": (19456, 2560, SILU)}.items():
        x = R.randn_bf16((M, K), 9300 + M + K)
        w = R.randn_bf16((N, K), 9301 + N, 0.02)
        cfgs = [dict(kernel=_lib.KERNEL_VALU, n_tiles=2, waves=8, unroll=5, splits=1),
                dict(kernel=_lib.KERNEL_VALU, n_tiles=4, waves=4, unroll=4, splits=2),
                dict(kernel=_lib.KERNEL_VALU, n_tiles=2, waves=5, unroll=4, splits=1),
                dict(kernel=_lib.KERNEL_VALU, n_tiles=4, waves=6, unroll=5, splits=1),
                dict(kernel=_lib.KERNEL_VALU, n_tiles=1, waves=3, unroll=2, splits=3)]
        if name == "down":
            cfgs.append(dict(kernel=_lib.KERNEL_VALU, n_tiles=1, waves=8, unroll=10, splits=1))
            cfgs.append(dict(kernel=_lib.KERNEL_VALU, n_tiles=2, waves=8, unroll=3, splits=4))
        _run_configs(x, w, epi, cfgs)


@pytest.mark.parametrize("M", [1, 8, 33, 64])
def test_stream_persistent_many_blocks(device, M):
    """More blocks than workgroups: every workgroup walks several blocks while
    the ring streams across block boundaries (lm_head-like width)."""
    K, N = 2560, 16 * 256 * 3 + 40
    x = R.randn_bf16((M, K), 9000 + M)
    w = R.randn_bf16((N, K), 9001, 0.02)
    for cfg in (dict(kernel=_lib.KERNEL_STREAM, splits=1, unroll=4), dict(kernel=_lib.KERNEL_STREAM, splits=2, unroll=5)):
        check_linear(x, w, f"stream persistent M={M}", cfg)


def test_split_count_only_changes_summation_order(device):
    x = R.randn_bf16((1, 4096), 8300)
    w = R.randn_bf16((2560, 4096), 8301, 0.02)
    exact, mag = R.linear_exact(x, w)
    outs = []
    for sp in (1, 2, 4, 8, 16):
        cfg = dict(kernel=_lib.KERNEL_MFMA, splits=sp)
        say("splits", sp)
        y = krk(x, w, NONE, cfg)
        assert R.within_fp32_bound(y, exact, mag, 4096).all()
        outs.append(y)
    # splits=1 twice is bit-identical; other counts differ at most by rounding order
    assert torch.equal(krk(x, w, NONE, dict(kernel=_lib.KERNEL_MFMA, splits=1)), outs[0])


# ---------------------------------------------------------------- runtime contract


def test_graph_capture_and_replay(device):
    """Calls (including split-K ones with their self-resetting counters) are
    captured in one graph and replayed several times, with eager work and
    synchronisation between replays; every replay matches the eager result."""
    shapes = [(1, 6144, 2560, NONE), (1, 2560, 4096, NONE), (8, 19456, 2560, SILU), (64, 2560, 9728, NONE),
              (1, 2560, 9728, NONE), (48, 19456, 2560, SILU), (64, 20000, 2560, NONE)]
    mms, ins = [], []
    for i, (M, N, K, epi) in enumerate(shapes):
        cls = G.SkinnyGateUp(M, N // 2, K, device) if epi == SILU else G.SkinnyMatmul(M, N, K, device)
        mms.append(cls)
        ins.append((R.randn_bf16((M, K), 8400 + i).to(device), R.randn_bf16((N, K), 8500 + i, 0.02).to(device)))
    say("graph", shapes)
    eager = [mm(a, w).clone() for mm, (a, w) in zip(mms, ins)]
    outs = [torch.empty_like(e) for e in eager]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for mm, (a, w), o in zip(mms, ins, outs):
            mm.run(a, w, o)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for mm, (a, w), o in zip(mms, ins, outs):
            mm.run(a, w, o)
    for rep in range(4):
        for o in outs:
            o.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for e, o in zip(eager, outs):
            assert torch.equal(e, o), f"replay {rep} differs from eager"
        _ = mms[1](*ins[1])  # eager call between replays shares the workspace
        torch.cuda.synchronize()


def test_alias_and_shape_errors_on_gpu(device):
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=device)
    w = torch.zeros(64, 256, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="may not share"):
        G.gemm_into(x, w, x[:, :64])
    with pytest.raises(ValueError):
        G.SkinnyMatmul(4, 64, 256, device)(x, torch.zeros(64, 128, dtype=torch.bfloat16, device=device))


def test_pickers_return_validated_callables(device):
    a = R.randn_bf16((8, 2560), 8600).to(device)
    w = R.randn_bf16((6144, 2560), 8601, 0.02).to(device)
    wgu = R.randn_bf16((2 * 9728, 2560), 8602, 0.02).to(device)
    logs = []
    say("pickers")
    mm = G.pick_matmul(a, w, log=logs.append)
    gu = G.pick_gateup(a, wgu, log=logs.append)
    assert_parity(mm(a, w).cpu(), R.linear_bf16(a, w), "pick_matmul")
    assert_parity(gu(a, wgu).cpu(), R.gateup_bf16(a, wgu), "pick_gateup")
    assert_parity(gu(a, wgu[:9728], wgu[9728:]).cpu(), R.gateup_bf16(a, wgu), "pick_gateup halves")
    assert any("us" in l for l in logs)


@pytest.mark.parametrize("M", [1, 2, 4])
def test_gemv_wrapper(device, M):
    """Gemv (reference engine/kernels/gemm.py:248-281): plain; gateup=True
    with the gate and up weights as the two halves of one tensor or as the
    whole tensor; and every one of the reference's GEMV_CONFIGS
    (gemm.py:284-288) through the Triton-argument constructor."""
    K, N, I = 2560, 6144, 1216
    x = R.randn_bf16((M, K), 9300 + M)
    w = R.randn_bf16((N, K), 9301, 0.02)
    wgu = R.randn_bf16((2 * I, K), 9302, 0.02)
    xd, wd, wgud = x.to(device), w.to(device), wgu.to(device)
    say("Gemv", M)
    assert_parity(G.Gemv(M, N, K, device)(xd, wd).cpu(), R.linear_bf16(x, w), f"Gemv M={M}")
    gu = G.Gemv(M, I, K, device, gateup=True)
    halves = gu(xd, wgud[:I], wgud[I:]).cpu()
    assert_parity(halves, R.gateup_bf16(x, wgu), f"Gemv gateup M={M}")
    assert torch.equal(gu(xd, wgud).cpu(), halves)
    with pytest.raises(ValueError):
        gu(xd, wgud[:I], wgud[I:].clone())  # not the two halves of one weight
    for cfg in ({"block_n": 32, "block_k": 256, "split_k": 1, "num_warps": 4, "num_stages": 3},
                {"block_n": 32, "block_k": 256, "split_k": 4, "num_warps": 4, "num_stages": 3},
                {"block_n": 16, "block_k": 256, "split_k": 8, "num_warps": 2, "num_stages": 3}):
        say("Gemv reference config", cfg)
        assert_parity(G.Gemv(M, N, K, device, **cfg)(xd, wd).cpu(), R.linear_bf16(x, w), f"Gemv {cfg}")
        g2 = G.Gemv(M, I, K, device, gateup=True, **cfg)
        assert_parity(g2(xd, wgud[:I], wgud[I:]).cpu(), R.gateup_bf16(x, wgu), f"Gemv gateup {cfg}")


@pytest.mark.parametrize("M", [8, 16, 32])
def test_reference_constructor_configs(device, M):
    """SkinnyMatmul / SkinnyGateUp built from the reference's CONFIGS
    (engine/kernels/gemm.py:364-375) run the translated configuration and
    match the oracle."""
    K, N, I = 2560, 768, 1216
    x = R.randn_bf16((M, K), 9400 + M)
    w = R.randn_bf16((N, K), 9401, 0.02)
    wgu = R.randn_bf16((2 * I, K), 9402, 0.02)
    xd, wd, wgud = x.to(device), w.to(device), wgu.to(device)
    ref, ref_gu = R.linear_bf16(x, w), R.gateup_bf16(x, wgu)
    for cfg in ({"block_n": 64, "block_k": 128, "split_k": 1, "num_warps": 4, "num_stages": 3},
                {"block_n": 64, "block_k": 64, "split_k": 4, "num_warps": 4, "num_stages": 4},
                {"block_n": 32, "block_k": 64, "split_k": 8, "num_warps": 4, "num_stages": 4},
                {"block_n": 32, "block_k": 128, "split_k": 2, "num_warps": 4, "num_stages": 3, "persist": 2}):
        mm = G.SkinnyMatmul(M, N, K, device, **cfg)
        say("reference config", M, cfg, mm.resolved_config)
        assert_parity(mm(xd, wd).cpu(), ref, f"SkinnyMatmul {cfg}")
        gu = G.SkinnyGateUp(M, I, K, device, **cfg)
        assert_parity(gu(xd, wgud[:I], wgud[I:]).cpu(), ref_gu, f"SkinnyGateUp {cfg}")


# ------------------------------------------------------------------ warm-up tuner

_TUNE_SHAPES = {"qkv": (2560, 6144, NONE), "o": (4096, 2560, NONE), "gate_up": (2560, 19456, SILU),
                "down": (9728, 2560, NONE), "lm_head": (2560, 151936, NONE)}


@pytest.mark.parametrize("shape,M", [("qkv", 8), ("gate_up", 4), ("down", 32), ("o", 64), ("lm_head", 1),
                                     ("gate_up", 64)])
def test_tune_validates_every_candidate(device, shape, M):
    """The tuner runs every candidate configuration at a real shape: each
    must pass the acceptance rules (a rejection is a kernel bug; gate_up at
    M = 64 also meets the reference's pointwise M = 64 rule on every weight
    of a 6-weight rotation), the winner is no slower than the table's plan,
    and a second tuning of the shape comes from the cache."""
    from kernels import tune as T
    K, N, epi = _TUNE_SHAPES[shape]
    a = R.randn_bf16((M, K), 9600 + M).to(device)
    ws = [R.randn_bf16((N, K), 9601 + i, 0.02).to(device) for i in range(6 if (shape, M) == ("gate_up", 64) else 2)]
    cache = T.TuneCache()
    say("tune", shape, M, len(T.candidates(M, N, K, epi)), "candidates")
    r = G.tune_projection(a, ws[0], epi, ws=ws, cache=cache)
    bad = [(t.config, t.note) for t in r.trials if t.us is None]
    assert not bad, f"candidates rejected or failed: {bad[:3]}"
    assert len(r.trials) == len(T.candidates(M, N, K, epi))
    assert r.trials[0].config == G.plan(M, N, K, epi) and r.plan_us is not None
    assert r.us <= r.plan_us
    again = G.tune_projection(a, ws[0], epi, ws=ws, cache=cache)
    assert again.cached and again.config == r.config
    mm = G.SkinnyGateUp(M, N // 2, K, device, config=r.config) if epi == SILU else G.SkinnyMatmul(M, N, K, device, config=r.config)
    ref = R.gateup_bf16(a.cpu(), ws[1].cpu()) if epi == SILU else R.linear_bf16(a.cpu(), ws[1].cpu())
    assert_parity(mm(a, ws[1]).cpu(), ref, f"tuned {shape} M={M}")


def test_tune_budget_cache_file_and_normed(device, tmp_path):
    """An expired budget measures only the plan; results persist to the JSON
    cache file and load in a new cache; normed tuning validates xout too."""
    from kernels import budget, tune as T
    M, K, N = 2, 2560, 6144
    a = R.randn_bf16((M, K), 9700).to(device)
    w = R.randn_bf16((N, K), 9701, 0.02).to(device)
    path = str(tmp_path / "tuned.json")
    budget.start(0.0)
    try:
        r = G.tune_projection(a, w, NONE, cache=T.TuneCache(path))
    finally:
        budget.clear()
    assert len(r.trials) == 1 and r.config == G.plan(M, N, K, NONE)
    loaded = T.TuneCache(path)
    assert loaded.get(T.TuneCache.key(device, "matmul", M, N, K)) == r.config
    x, y, wn = (t.to(device) for t in _norm_inputs(M, K, 9702))
    rn = G.tune_projection(x, w, NONE, cache=T.TuneCache(), norm=(y, wn, EPS), limit=12)
    assert len(rn.trials) == 12 and all(t.us is not None for t in rn.trials), [t.note for t in rn.trials]
    f = G.pick_normed("matmul", x, y, wn, w, EPS, cache=T.TuneCache(), tune=True)
    xo = torch.empty_like(x)
    out = f(x, y, wn, xo, w)
    torch.cuda.synchronize()
    _check_normed(x.cpu(), y.cpu(), wn.cpu(), w.cpu(), NONE, xo.cpu(), out.cpu(), "tuned pick_normed")


# ------------------------------------------------------------------ normed projections (RMSNorm prologue)

EPS = 1e-6
#: (K, N, epilogue) of the normed projections (their input is rms_norm(x + y)).
QWEN = {"qkv": (2560, 6144, NONE), "gate_up": (2560, 19456, SILU), "lm_head": (2560, 151936, NONE)}


def krk_normed(x, y, wn, w, epilogue=NONE, config=None, device="cuda:0", ws=None, with_ws=False):
    """Normed HIP call on CPU bf16 inputs; returns (xout, out) on the CPU
    (and the workspace with ``with_ws``).  Outputs start NaN-filled."""
    M, K = x.shape
    N = w.shape[0]
    nout = N // 2 if epilogue == SILU else N
    xd, yd, gd, wd = x.to(device), y.to(device), wn.to(device), w.to(device)
    out = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device=device)
    xout = torch.full((M, K), float("nan"), dtype=torch.bfloat16, device=device)
    if ws is None:
        nbytes = G.workspace_bytes(M, N, K, epilogue, config, normed=True)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes else None
    G.gemm_into(xd, wd, out, epilogue, ws, config, norm=(yd, gd, xout, EPS))
    torch.cuda.synchronize()
    if with_ws:
        return xout.cpu(), out.cpu(), ws
    return xout.cpu(), out.cpu()


def _norm_inputs(M, K, seed):
    return (R.randn_bf16((M, K), seed), R.randn_bf16((M, K), seed + 1, 0.5), R.randn_bf16((K,), seed + 2))


def _check_normed(x, y, wn, w, epi, got_xout, got, what):
    ref_xout, ref = (R.normed_gateup_bf16 if epi == SILU else R.normed_linear_bf16)(x, y, wn, EPS, w)
    assert torch.equal(got_xout, ref_xout), f"{what}: xout differs from bf16(x + y)"
    assert_parity(got, ref, what)


@pytest.mark.parametrize("shape,M", [("qkv", M) for M in (1, 2, 3, 4, 8, 9, 32, 64)] +
                                    [("gate_up", M) for M in (1, 2, 5, 8, 16, 32, 64)] +
                                    [("lm_head", M) for M in (1, 4, 8, 32)])
def test_normed_qwen_shapes(device, shape, M):
    K, N, epi = QWEN[shape]
    x, y, wn = _norm_inputs(M, K, 9300 + M)
    w = R.randn_bf16((N, K), 9310 + M, 0.02)
    say("normed", shape, M, "fused" if G.normed_fused(M, N, K, epi) else "prologue")
    xo, out = krk_normed(x, y, wn, w, epi)
    _check_normed(x, y, wn, w, epi, xo, out, f"normed {shape} M={M}")


@pytest.mark.parametrize("M,N,K,epi", [(1, 6144, 2560, NONE), (1, 19456, 2560, SILU), (1, 520, 2056, NONE),
                                       (1, 96, 1000, SILU), (4, 6144, 2560, NONE), (7, 96, 1000, SILU)])
def test_normed_fused_and_prologue_paths_agree(device, M, N, K, epi):
    """The fused VALU prologue (every W-rows-per-wave choice, split and
    unsplit K, ragged K), the VALU plan behind the prologue kernel, and an
    MFMA plan behind it are all within tolerance of the oracle, and the fused
    call is deterministic."""
    x, y, wn = _norm_inputs(M, K, 9400 + M)
    w = R.randn_bf16((N, K), 9410, 0.02)
    cfgs = [dict(kernel=_lib.KERNEL_VALU, unroll=5, n_tiles=nt, splits=sp) for nt in (1, 2, 4) for sp in (1, 2)]
    cfgs += [dict(kernel=_lib.KERNEL_VALU, unroll=2, splits=1), dict(kernel=_lib.KERNEL_MFMA_LDS, splits=1)]
    ran = 0
    for cfg in cfgs:
        try:
            fused = G.normed_fused(M, N, K, epi, cfg)
        except ValueError:
            continue
        say("normed config", M, N, K, epi, cfg, fused)
        xo, out = krk_normed(x, y, wn, w, epi, cfg)
        _check_normed(x, y, wn, w, epi, xo, out, f"normed {cfg}")
        if fused:
            assert torch.equal(out, krk_normed(x, y, wn, w, epi, cfg)[1])
        ran += 1
    assert ran >= 3


@pytest.mark.parametrize("shape,M", [("qkv", M) for M in (1, 2, 3, 4)] + [("gate_up", M) for M in (1, 2)] +
                                    [("lm_head", M) for M in (1, 2)])
def test_normed_fused_plans_and_separate_prologue(device, shape, M):
    """Normed plans that fuse the prologue (one launch) and the same
    configuration behind the separate prologue kernel (prologue = 1) both
    match the oracle's reference-rounded normed projection, with xout
    bit-exact; a second fused call with other inputs on the same workspace
    is correct too, and the fused call is deterministic."""
    K, N, epi = QWEN[shape]
    plan = G.normed_plan(M, N, K, epi)
    assert G.normed_fused(M, N, K, epi), "the normed plan fuses the prologue at this M"
    w = R.randn_bf16((N, K), 9320 + M, 0.02)
    ws = None
    for rep in range(2):
        x, y, wn = _norm_inputs(M, K, 9330 + 10 * rep + M)
        say("normed fused", shape, M, rep, plan)
        xo, out, ws = krk_normed(x, y, wn, w, epi, ws=ws, with_ws=True)
        _check_normed(x, y, wn, w, epi, xo, out, f"normed fused {shape} M={M} call {rep}")
    assert torch.equal(out, krk_normed(x, y, wn, w, epi, ws=ws)[1]), "fused normed call not deterministic"
    sep = dict(plan, prologue=1)
    assert not G.normed_fused(M, N, K, epi, sep)
    say("normed separate prologue", shape, M, sep)
    xo2, out2 = krk_normed(x, y, wn, w, epi, sep)
    _check_normed(x, y, wn, w, epi, xo2, out2, f"normed prologue kernel {shape} M={M}")


@pytest.mark.parametrize("M,N,K,epi,splits", [
    (5, 600, 2560, NONE, 1), (16, 2 * 300, 2560, SILU, 1), (17, 1000, 1000, NONE, 1), (20, 2 * 200, 2056, SILU, 1),
    (32, 2 * 600, 2560, SILU, 1), (33, 520, 2560, NONE, 1), (48, 2 * 96, 1032, SILU, 1), (64, 1000, 2560, NONE, 1),
    (20, 600, 2560, NONE, 2), (40, 2 * 300, 5120, SILU, 2), (64, 520, 4096, NONE, 3), (100, 600, 2560, NONE, 1)])
def test_normed_stream_fragment_order(device, M, N, K, epi, splits):
    """Normed calls on the stream kernel, whose prologue writes the
    normalised rows in the kernel's MFMA fragment order (rows past M and k
    past K up to whole 512-k stages zero): one to four 16-row tiles, ragged
    K (down to an 8-element last stage) and N, split K, two ring depths, and
    past 64 rows the row-major path.  xout bit-exact, outputs against the
    oracle, and a second call with other inputs on the same workspace (which
    the first left holding the previous rows)."""
    w = R.randn_bf16((N, K), 9510 + N, 0.02)
    for depth in (3, 5):
        cfg = dict(kernel=_lib.KERNEL_STREAM, splits=splits, unroll=depth)
        ws = None
        for rep in range(2):
            x, y, wn = _norm_inputs(M, K, 9500 + M + 10 * rep)
            say("normed stream", M, N, K, epi, cfg, rep)
            xo, out, ws = krk_normed(x, y, wn, w, epi, cfg, ws=ws, with_ws=True)
            _check_normed(x, y, wn, w, epi, xo, out, f"normed stream {cfg} M={M} call {rep}")


def _normed_fused_configs(M, epi):
    """VALU configurations at the fused depth (M <= 8): every W-rows-per-wave
    and wave count (those with fewer waves than 512-k blocks do not fuse);
    LDS-staged ones (M <= 32): one or two weight tiles, two or three stages
    in flight (those that do not fuse are skipped), the tiles' full channel
    count and 8 fewer."""
    cfgs = []
    if M <= 8:
        for nt, wv in itertools.product((1, 2, 4), (2, 4, 5, 8)):
            if epi == SILU and nt == 1:
                continue
            cfgs.append(dict(kernel=_lib.KERNEL_VALU, n_tiles=nt, waves=wv, unroll=5, splits=1))
    for nt, pf in itertools.product((1, 2), (2, 3)):
        if epi == SILU and nt == 1:
            continue
        full = 16 * (nt // 2 if epi == SILU else nt)
        for ch in sorted({full, max(8, full - 8)}):
            cfgs.append(dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=nt, unroll=pf, k_chunk=512, splits=1, channels=ch))
    return cfgs


@pytest.mark.parametrize("M,N,K,epi", [(3, 1040, 2560, NONE), (5, 600, 2048, SILU), (8, 2064, 1000, NONE),
                                       (6, 496, 2560, SILU), (8, 4100, 2560, NONE), (1, 96, 1000, SILU),
                                       (7, 520, 2056, NONE), (2, 6144, 2560, NONE), (4, 19456, 2560, SILU),
                                       (9, 1040, 2560, NONE), (12, 600, 2048, SILU), (16, 2064, 1000, NONE),
                                       (13, 6144, 2560, NONE), (16, 19456, 2560, SILU), (11, 520, 2056, NONE),
                                       (15, 4100, 512, SILU), (24, 1040, 2560, NONE), (32, 6144, 2560, NONE),
                                       (20, 600, 2048, SILU), (29, 520, 1000, NONE)])
def test_normed_fused_configs(device, M, N, K, epi):
    """The fused prologue under every fusing configuration (VALU at M <= 8,
    LDS-staged MFMA at M <= 32), ragged K and N, K of one to five 512-k
    stages, both epilogues, against the oracle; deterministic."""
    x, y, wn = _norm_inputs(M, K, 9800 + M)
    w = R.randn_bf16((N, K), 9810 + M, 0.02)
    ran = 0
    for cfg in _normed_fused_configs(M, epi):
        try:
            fused = G.normed_fused(M, N, K, epi, cfg)
        except ValueError:
            continue  # a combination the library does not provide
        if not fused:
            continue
        say("normed fused config", M, N, K, epi, cfg)
        xo, out, ws = krk_normed(x, y, wn, w, epi, cfg, with_ws=True)
        _check_normed(x, y, wn, w, epi, xo, out, f"normed fused {cfg}")
        assert torch.equal(out, krk_normed(x, y, wn, w, epi, cfg, ws=ws)[1])
        ran += 1
    assert ran >= 1


@pytest.mark.parametrize("M,shape", [(1, "qkv"), (2, "gate_up"), (4, "qkv"), (2, "lm_head"), (8, "gate_up"),
                                     (12, "qkv"), (16, "gate_up"), (9, "lm_head"), (24, "qkv"), (32, "gate_up")])
def test_normed_fused_special_values(device, M, shape):
    """Rows with a NaN in d, an inf in x, s = x + d all zero (rstd =
    1/sqrt(eps)) and a -0 row: the fused call's NaN pattern and finite values
    match the oracle's reference-rounded chain (VALU fusion at M <= 8, the
    LDS-staged kernel's above)."""
    K, N, epi = QWEN[shape]
    if G.normed_fused(M, N, K, epi):
        cfg = G.normed_plan(M, N, K, epi)
    elif M <= 8:
        cfg = dict(kernel=_lib.KERNEL_VALU, n_tiles=2, unroll=5, waves=8, splits=1)
    else:
        cfg = dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=2, unroll=2, k_chunk=512, splits=1)
    if shape == "lm_head":
        N = 4096  # lm_head's plan at its K, fewer rows to check
    assert G.normed_fused(M, N, K, epi, cfg)
    x, y, wn = _norm_inputs(M, K, 9900 + M)
    y[0, 17] = float("nan")
    if M > 1:
        x[1, 100] = float("inf")
    if M > 2:
        y[2] = -x[2]
    if M > 3:
        x[3] = -0.0
        y[3] = -0.0
    w = R.randn_bf16((N, K), 9910 + M, 0.02)
    say("normed fused special", shape, M, cfg)
    xo, out = krk_normed(x, y, wn, w, epi, cfg)
    ref_xout, ref = (R.normed_gateup_bf16 if epi == SILU else R.normed_linear_bf16)(x, y, wn, EPS, w)
    assert torch.equal(xo.view(torch.int16), ref_xout.view(torch.int16)) or torch.equal(
        torch.isnan(xo), torch.isnan(ref_xout)) and torch.equal(xo.nan_to_num(0), ref_xout.nan_to_num(0)), "xout"
    assert torch.equal(torch.isnan(out), torch.isnan(ref)), "NaN pattern differs from the oracle's"
    assert torch.isnan(out[0]).all(), "a NaN in d poisons its row"
    if M > 1:
        assert torch.isnan(out[1]).all(), "an inf in x gives rstd 0 and NaN (inf * 0) in its row"
    fin = ~torch.isnan(ref)
    bad = (out.float()[fin] - ref.float()[fin]).abs() > 2e-2 + 1e-2 * ref.float()[fin].abs()
    assert not bad.any(), f"{int(bad.sum())} finite values outside 2e-2 + 1e-2|ref|"


def test_normed_rows_beyond_64(device):
    M, N, K = 100, 384, 2560
    x, y, wn = _norm_inputs(M, K, 9500)
    w = R.randn_bf16((N, K), 9501, 0.02)
    xo, out = krk_normed(x, y, wn, w)
    _check_normed(x, y, wn, w, NONE, xo, out, "normed M=100")


@pytest.mark.parametrize("M,K", [(1, 2560), (7, 512), (64, 2560), (3, 16384), (5, 2056)])
def test_add_rms_norm_kernel(device, M, K):
    x, y, wn = _norm_inputs(M, K, 9600 + M)
    ref_xo, ref_n = R.add_rms_norm_bf16(x, y, wn, EPS)
    xd = x.to(device)
    out = G.add_rms_norm(xd, y.to(device), wn.to(device), EPS, xout=torch.empty_like(xd))
    xo2 = xd.clone()
    out_inplace = G.add_rms_norm(xo2, y.to(device), wn.to(device), EPS)  # xout = x (in place)
    torch.cuda.synchronize()
    assert torch.equal(xo2.cpu(), ref_xo)
    for got in (out.cpu(), out_inplace.cpu()):
        gb, rb = R.to_bits(got).astype(np.int32), R.to_bits(ref_n).astype(np.int32)
        assert np.abs(gb - rb).max() <= 1 and (gb == rb).mean() > 0.999
    assert torch.equal(out.cpu(), out_inplace.cpu())


def test_normed_graph_replay(device):
    """Fused and prologue-kernel normed calls captured in one graph replay to
    the eager results, with eager work between replays."""
    lds_fused = {"kernel": _lib.KERNEL_MFMA_LDS, "n_tiles": 2, "k_chunk": 512, "splits": 1}
    cases = [(1, 6144, 2560, NONE, None), (8, 19456, 2560, SILU, None), (32, 6144, 2560, NONE, None),
             (32, 19456, 2560, SILU, None), (32, 19456, 2560, SILU, {"kernel": _lib.KERNEL_STREAM, "prologue": 1}),
             (64, 151936, 2560, NONE, None), (2, 19456, 2560, SILU, None), (4, 6144, 2560, NONE, None),
             (12, 6144, 2560, NONE, lds_fused), (16, 19456, 2560, SILU, lds_fused),
             (32, 6144, 2560, NONE, dict(lds_fused, unroll=2))]
    ops, ins, eager, outs = [], [], [], []
    for i, (M, N, K, epi, cfg) in enumerate(cases):
        op = (G.SkinnyGateUp(M, N // 2, K, device, config=cfg) if epi == SILU
              else G.SkinnyMatmul(M, N, K, device, config=cfg))
        x, y, wn = (t.to(device) for t in _norm_inputs(M, K, 9700 + i))
        w = R.randn_bf16((N, K), 9710 + i, 0.02).to(device)
        xo = torch.empty_like(x)
        ops.append(op)
        ins.append((x, y, wn, w, xo))
        eager.append(op(x, w, norm=(y, wn, xo, EPS)).clone())
        outs.append(torch.empty_like(eager[-1]))
    torch.cuda.synchronize()
    say("normed graph", cases)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for op, (x, y, wn, w, xo), o in zip(ops, ins, outs):
            op.run(x, w, o, norm=(y, wn, xo, EPS))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for op, (x, y, wn, w, xo), o in zip(ops, ins, outs):
            op.run(x, w, o, norm=(y, wn, xo, EPS))
    for rep in range(3):
        for o in outs:
            o.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for e, o in zip(eager, outs):
            assert torch.equal(e, o), f"normed replay {rep} differs from eager"
        _ = ops[0](ins[0][0], ins[0][3])  # eager plain call between replays shares the workspace
        torch.cuda.synchronize()


def test_pick_normed_returns_validated_callable(device):
    M, K, N = 4, 2560, 6144
    x, y, wn = (t.to(device) for t in _norm_inputs(M, K, 9800))
    w = R.randn_bf16((N, K), 9801, 0.02).to(device)
    logs = []
    f = G.pick_normed("matmul", x, y, wn, w, EPS, log=logs.append)
    xo = torch.empty_like(x)
    out = f(x, y, wn, xo, w)
    torch.cuda.synchronize()
    _check_normed(x.cpu(), y.cpu(), wn.cpu(), w.cpu(), NONE, xo.cpu(), out.cpu(), "pick_normed")
    assert any("normed matmul" in l for l in logs)
    wgu = R.randn_bf16((2 * 9728, K), 9802, 0.02).to(device)
    g = G.pick_normed("gateup", x, y, wn, wgu, EPS)
    assert g(x, y, wn, xo, wgu).shape == (M, 9728)


# ------------------------------------------------------------------ token selection (lm_head argmax / top-k)

def krk_select(x, w, k, config=None, logits=True, device="cuda:0", wd=None):
    """Selecting HIP call on CPU inputs; returns (idx, vals, logits or None) on the CPU."""
    M, K = x.shape
    N = w.shape[0]
    op = G.SkinnySelect(M, N, K, device, k, config)
    xd = x.to(device)
    wd = w.to(device) if wd is None else wd
    lg = torch.empty((M, N), dtype=torch.bfloat16, device=device) if logits else None
    vals = torch.empty((M, k), dtype=torch.bfloat16, device=device)
    idx = torch.empty((M, k), dtype=torch.int64, device=device)
    op.run(xd, wd, idx, lg, vals)
    torch.cuda.synchronize()
    return idx.cpu(), vals.cpu(), (lg.cpu() if logits else None)


def _check_selection(idx, vals, logits, k, what):
    """Bit-exact: the selection equals the oracle's top-k of the same logits."""
    ref_idx, ref_vals = R.topk_rows(logits, k)
    if not torch.equal(idx, ref_idx):
        rows = (idx != ref_idx).any(dim=1).nonzero().flatten().tolist()
        pytest.fail(f"{what}: selection differs on rows {rows[:5]}: got {idx[rows[0]].tolist()} "
                    f"want {ref_idx[rows[0]].tolist()}")
    # A NaN is reported as the canonical quiet NaN; every other value bit for bit.
    gb, rb = R.to_bits(vals), R.to_bits(ref_vals)
    gnan, rnan = (gb & 0x7FFF) > 0x7F80, (rb & 0x7FFF) > 0x7F80
    assert np.array_equal(gnan, rnan) and np.array_equal(gb[~gnan], rb[~rnan]), f"{what}: selected values differ"


@pytest.fixture(scope="module")
def lm_head_dev(lm_head):
    return lm_head.to("cuda:0")


@pytest.mark.parametrize("k", [1, 8])
@pytest.mark.parametrize("M", [1, 2, 4, 5, 8, 16, 17, 32, 64, 100])
def test_select_lm_head(device, lm_head, lm_head_dev, M, k):
    x = R.randn_bf16((M, R.HIDDEN), R.seed_for(5, M, "x") + 7)
    say("select lm_head", M, k, G.select_plan(M, R.VOCAB, R.HIDDEN))
    idx, vals, logits = krk_select(x, lm_head, k, wd=lm_head_dev)
    _check_selection(idx, vals, logits, k, f"select M={M} k={k}")
    ref = R.linear_bf16(x, lm_head)
    assert_parity(logits, ref, f"select logits M={M}")
    if k == 1:
        assert torch.equal(idx[:, 0], R.argmax_rows(ref)), f"select M={M}: argmax differs from the oracle's"
    idx2, vals2, _ = krk_select(x, lm_head, k, logits=False, wd=lm_head_dev)
    assert torch.equal(idx, idx2) and torch.equal(vals.view(torch.int16), vals2.view(torch.int16)), \
        "selection without logits differs"


@pytest.mark.parametrize("M", [5, 16])
def test_select_lm_head_fused_lds(device, lm_head, lm_head_dev, M):
    """Argmax fused into an LDS-staged MFMA lm_head projection (a tuned
    choice at these M; the table's plan there is the stream kernel)."""
    cfg = dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=2, unroll=3, k_chunk=256, splits=1)
    assert G.select_fused(M, R.VOCAB, R.HIDDEN, 1, cfg)
    x = R.randn_bf16((M, R.HIDDEN), R.seed_for(5, M, "x") + 9)
    say("select lm_head fused lds", M)
    idx, vals, logits = krk_select(x, lm_head, 1, cfg, wd=lm_head_dev)
    _check_selection(idx, vals, logits, 1, f"select fused lds M={M}")
    ref = R.linear_bf16(x, lm_head)
    assert_parity(logits, ref, f"select fused lds logits M={M}")
    assert torch.equal(idx[:, 0], R.argmax_rows(ref)), f"select fused lds M={M}: argmax differs from the oracle's"


def _tie_weights(N, K, seed):
    """W whose rows repeat: row 3·i + j = row 3·i for j < 3, so equal logits
    sit at consecutive indices; one row pair is NaN-producing."""
    base = R.randn_bf16((-(-N // 3), K), seed, 0.02)
    w = base.repeat_interleave(3, dim=0)[:N].clone()
    return w


@pytest.mark.parametrize("M,N,K", [(1, 1000, 2560), (3, 4099, 2560), (4, 300, 2560), (7, 1000, 512),
                                   (33, 5000, 2560), (64, 257, 1024), (2, 600001, 64)])
def test_select_ties_nan_and_configs(device, M, N, K):
    """Equal logits (repeated W rows) rank the lower index first; a NaN logit
    ranks above everything; every projection configuration, fused or not,
    with or without caller logits, selects the same indices bit for bit.
    N = 600001 has more than 32 chunks of logits per row, so a row's chunk
    lists exceed the LDS ranking and merge through sorted-list trees."""
    x = R.randn_bf16((M, K), 9900 + M)
    w = _tie_weights(N, K, 9901 + N)
    w[N // 2, 0] = float("nan")         # logits of row N//2 are NaN in every row m
    cfgs = [None]
    if M <= 4 and K == 2560:
        cfgs += [dict(kernel=_lib.KERNEL_VALU, unroll=5, n_tiles=nt, waves=wv, splits=1)
                 for nt in (1, 2, 4) for wv in (1, 4, 8)]
    cfgs += [dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=nt, unroll=pf, k_chunk=256, splits=1)
             for nt in (2, 4) for pf in (2, 3)]
    cfgs += [dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=2, unroll=2, k_chunk=256, splits=1, channels=24)]
    cfgs += [dict(kernel=_lib.KERNEL_STREAM), dict(kernel=_lib.KERNEL_VALU, splits=2),
             dict(kernel=_lib.KERNEL_MFMA, splits=1)]
    base = {}
    for cfg in cfgs:
        for k in (1, 3, 8):
            say("select ties", M, N, K, k, cfg)
            try:
                idx, vals, logits = krk_select(x, w, k, cfg)
            except ValueError as e:  # a combination the library does not provide (e.g. unroll 3 on big tiles)
                assert cfg is not None and "invalid token selection" in str(e), e
                continue
            _check_selection(idx, vals, logits, k, f"select {cfg} k={k}")
            assert (idx[:, 0] == N // 2).all(), "the NaN logit must rank first"
            base.setdefault(k, idx)
            assert torch.equal(idx, base[k]), f"select {cfg} k={k}: differs from the first configuration"
            idx2, vals2, _ = krk_select(x, w, k, cfg, logits=False)
            assert torch.equal(idx, idx2) and torch.equal(vals.view(torch.int16), vals2.view(torch.int16)), \
                f"select {cfg} k={k}: differs without logits"


def test_select_graph_replay(device, lm_head_dev):
    """Selecting calls captured in a graph replay to the eager result several
    times (their counters reset themselves), with eager work in between."""
    cases = [(1, 1), (8, 8), (32, 1)]
    ops, xs, eager, outs = [], [], [], []
    for i, (M, k) in enumerate(cases):
        op = G.SkinnySelect(M, R.VOCAB, R.HIDDEN, device, k)
        x = R.randn_bf16((M, R.HIDDEN), 9950 + i).to(device)
        ops.append(op)
        xs.append(x)
        eager.append(op(x, lm_head_dev).clone())
        outs.append(torch.empty_like(eager[-1]))
    torch.cuda.synchronize()
    say("select graph", cases)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for op, x, o in zip(ops, xs, outs):
            op.run(x, lm_head_dev, o)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for op, x, o in zip(ops, xs, outs):
            op.run(x, lm_head_dev, o)
    for rep in range(3):
        for o in outs:
            o.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for e, o in zip(eager, outs):
            assert torch.equal(e, o), f"select replay {rep} differs from eager"
        _ = ops[0](xs[0], lm_head_dev)
        torch.cuda.synchronize()
