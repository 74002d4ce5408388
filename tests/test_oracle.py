"""Pin the CPU oracle (oracle/gemm_ref.py, oracle/gemm_ref.c) to the mathematics.

The reference ships no golden vectors or kernel tests for this path (its one
test file, tests/test_client.py, mocks an HTTP client), so every oracle
function is pinned here by checks a plausible mistake cannot pass: fp64 brute
force with a rigorous fp32 error bound, exact integer-valued cases, special
values, an independent C restatement, and constructed ties.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gemm_ref as R

QWEN_K = (2560, 4096, 9728)
GOLDEN = Path(__file__).resolve().parent / "golden"


def _inputs(M, N, K, seed, xs=1.0):
    return R.randn_bf16((M, K), seed, xs), R.randn_bf16((N, K), seed + 1, 0.02)


@pytest.mark.parametrize("K", QWEN_K)
@pytest.mark.parametrize("M", [1, 8, 64])
def test_linear_within_fp32_bound_of_exact(M, K):
    """torch-CPU F.linear is an fp32-accumulated sum rounded once to bf16."""
    x, w = _inputs(M, 96, K, 100 + M + K)
    y = R.linear_bf16(x, w)
    exact, mag = R.linear_exact(x, w)
    ok = R.within_fp32_bound(y, exact, mag, K)
    assert ok.all(), f"{(~ok).sum()} elements outside the fp32 summation bound"
    # Most elements are the correctly rounded value: an fp32 order only moves
    # results that sit near a bf16 rounding boundary.
    mism = (R.to_bits(y) != R.f64_to_bf16_bits(exact)).mean()
    assert mism < 0.01, f"{mism:.4f} of elements differ from the correctly rounded result"


@pytest.mark.parametrize("K", QWEN_K)
def test_c_restatement_matches_exact_and_torch(K):
    x, w = _inputs(4, 64, K, 200 + K)
    ex_c, mag_c, y64 = R.c_linear_f64(x, w)
    ex_np, mag_np = R.linear_exact(x, w)
    np.testing.assert_allclose(ex_c, ex_np, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mag_c, mag_np, rtol=1e-12)
    assert np.array_equal(R.to_bits(y64), R.f64_to_bf16_bits(ex_np)), "C and numpy fp64->bf16 rounding differ"
    y32 = R.c_linear_f32(x, w)
    assert R.within_fp32_bound(y32, ex_np, mag_np, K).all()
    yt = R.linear_bf16(x, w)
    diff = np.abs(R.bits_to_f32(R.to_bits(y32)).astype(np.float64) - R.bits_to_f32(R.to_bits(yt)))
    assert (diff <= R.bf16_ulp(np.abs(ex_np)) * 1.0001 + R.fp32_sum_bound(mag_np, K) * 2).all()


def test_f64_to_bf16_single_rounding():
    """Values just above/below a bf16 midpoint that fp32 rounds onto the midpoint."""
    one = 1.0
    half_ulp = 2.0 ** -8  # bf16 ulp at 1.0 is 2^-7
    d = np.array([one + half_ulp + 2.0 ** -40, one + half_ulp - 2.0 ** -40, one + half_ulp,
                  -(one + half_ulp + 2.0 ** -40), 3 * half_ulp + one])
    got = R.f64_to_bf16_bits(d)
    want = np.array([0x3F81, 0x3F80, 0x3F80, 0xBF81, 0x3F82], np.uint16)
    assert np.array_equal(got, want), [hex(v) for v in got]


def test_f32_to_bf16_round_half_even_and_specials():
    f = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, np.inf, -np.inf, 0.0, -0.0, 3.4e38, np.nan], np.float32)
    got = R.f32_to_bf16_bits(f)
    assert list(got[:7]) == [0x3F80, 0x3F82, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x7F80]
    assert (got[7] & 0x7F80) == 0x7F80 and (got[7] & 0x7F) != 0
    # torch agrees on the finite cases
    t = torch.from_numpy(f[:7]).to(torch.bfloat16)
    assert np.array_equal(R.to_bits(t), got[:7])


def test_linear_integer_cases_are_exact():
    """Small-integer operands: every product and partial sum is exact, so the
    result is known exactly; a transposed operand, a dropped term or a sign
    error all change it."""
    M, N, K = 5, 7, 48
    m = np.arange(M)[:, None]
    n = np.arange(N)[:, None]
    k = np.arange(K)[None, :]
    xi = ((m + 1) * (k + 1)) % 7 - 3
    wi = ((n + 2) * (k + 3)) % 5 - 2
    want = xi @ wi.T
    assert np.abs(want).max() < 256  # exactly representable in bf16
    x = torch.from_numpy(xi.astype(np.float32)).bfloat16()
    w = torch.from_numpy(wi.astype(np.float32)).bfloat16()
    for y in (R.linear_bf16(x, w), R.c_linear_f32(x, w)):
        assert np.array_equal(y.float().numpy(), want.astype(np.float32))
    # the mistakes this rules out
    assert not np.array_equal((xi @ wi.T)[:, :-1], (xi[:, :-1] @ wi[:, :-1].T)[:, :-1])
    assert not np.array_equal(want, -want)


def test_linear_special_cases():
    K = 2560
    x, w = _inputs(3, 40, K, 300)
    z = torch.zeros_like(x)
    assert (R.linear_bf16(z, w).float() == 0).all()
    # one-hot rows pick one column of W^T exactly (a single bf16 product is exact)
    oh = torch.zeros_like(x)
    cols = [0, 1234, K - 1]
    for r, c in enumerate(cols):
        oh[r, c] = 1.0
    y = R.linear_bf16(oh, w)
    for r, c in enumerate(cols):
        assert torch.equal(y[r], w[:, c])
    # negation is exact, so it commutes with any summation order
    assert torch.equal(R.linear_bf16(-x, w), -R.linear_bf16(x, w))
    # identity block
    eye = torch.eye(40, K, dtype=torch.bfloat16)
    assert torch.equal(R.linear_bf16(x[:, :K], eye), x[:, :40])


def test_swiglu_matches_closed_form_and_c():
    g = R.randn_bf16((16, 512), 400, 3.0)
    u = R.randn_bf16((16, 512), 401, 2.0)
    gu = torch.cat([g, u], dim=1)
    out_t = R.swiglu_bf16(gu)
    out_c = R.c_swiglu(gu)
    gf = g.double().numpy()
    uf = u.double().numpy()
    s = R.bits_to_f32(R.f64_to_bf16_bits(gf / (1.0 + np.exp(-gf)))).astype(np.float64)
    closed = R.f64_to_bf16_bits(s * uf)
    for out in (out_t, out_c):
        b = R.to_bits(out)
        mism = b != closed
        assert mism.mean() < 2e-3
        of = R.bits_to_f32(b).astype(np.float64)
        cf = R.bits_to_f32(closed).astype(np.float64)
        assert (np.abs(of - cf) <= R.bf16_ulp(cf) * 1.0001).all()


def test_swiglu_has_three_roundings():
    """Find inputs where rounding once (silu·u in fp32, one rounding) differs
    from rounding three times; the oracle must give the three-rounding value."""
    rng = np.random.default_rng(5)
    g32 = rng.standard_normal(20000).astype(np.float32) * 3
    u32 = rng.standard_normal(20000).astype(np.float32) * 3
    gb = R.bits_to_f32(R.f32_to_bf16_bits(g32))
    ub = R.bits_to_f32(R.f32_to_bf16_bits(u32))
    s32 = gb / (np.float32(1) + np.exp(-gb))
    once = R.f32_to_bf16_bits(s32 * ub)
    thrice = R.f32_to_bf16_bits(R.bits_to_f32(R.f32_to_bf16_bits(s32)) * ub)
    idx = np.nonzero(once != thrice)[0]
    assert idx.size > 0
    g = torch.from_numpy(gb[idx]).bfloat16()[None]
    u = torch.from_numpy(ub[idx]).bfloat16()[None]
    out = R.swiglu_bf16(torch.cat([g, u], dim=1))
    agree_thrice = (R.to_bits(out)[0] == thrice[idx]).mean()
    assert agree_thrice > 0.99, agree_thrice
    c = np.array([R.c_lib().oracle_silu_mul1(int(a), int(b)) for a, b in zip(R.to_bits(g)[0], R.to_bits(u)[0])])
    assert (c == thrice[idx]).mean() > 0.99


def test_swiglu_gate_first_order():
    g = torch.tensor([[2.0, -1.0, 0.5]], dtype=torch.bfloat16)
    u = torch.tensor([[3.0, 4.0, -2.0]], dtype=torch.bfloat16)
    out = R.swiglu_bf16(torch.cat([g, u], dim=1))
    swapped = R.swiglu_bf16(torch.cat([u, g], dim=1))
    assert not torch.equal(out, swapped)
    want = (torch.nn.functional.silu(g.float()).bfloat16().float() * u.float()).bfloat16()
    assert torch.equal(out, want)


def test_swiglu_special_values():
    g = torch.tensor([[0.0, 100.0, -100.0, 20.0]], dtype=torch.bfloat16)
    u = torch.tensor([[5.0, 1.5, 7.0, -2.0]], dtype=torch.bfloat16)
    for out in (R.swiglu_bf16(torch.cat([g, u], 1)), R.c_swiglu(torch.cat([g, u], 1))):
        o = out.float()[0]
        assert o[0] == 0
        assert o[1] == 150.0          # silu(g) == g for large g
        assert abs(o[2]) < 1e-30      # silu(g) -> 0 for very negative g
        assert o[3] == -40.0


def test_gateup_c_restatement_agrees():
    x = R.randn_bf16((4, 2560), 500)
    w = R.randn_bf16((2 * 32, 2560), 501, 0.02)
    a = R.gateup_bf16(x, w)
    b = R.c_gateup_f32(x, w)
    assert R.close(b, a).all()
    assert (R.to_bits(a) != R.to_bits(b)).mean() < 0.02


def test_argmax_ties_lowest_index():
    data = np.load(GOLDEN / "argmax_ties.npz")
    exp = data["expected"]
    for i, e in enumerate(exp):
        row = R.from_bits(data[f"row{i}"])[None]
        assert R.argmax_rows(row).item() == e
        assert R.c_argmax_rows(row).item() == e


def test_argmax_random_rows_agree():
    v = R.randn_bf16((8, 151936), 600)
    assert torch.equal(R.argmax_rows(v), R.c_argmax_rows(v))


def test_seeded_inputs_reproducible():
    a = R.randn_bf16((3, 100), 7, 0.02)
    b = R.randn_bf16((3, 100), 7, 0.02)
    c = R.randn_bf16((3, 100), 8, 0.02)
    assert torch.equal(a, b) and not torch.equal(a, c)
    assert R.seed_for(4, 35, "down") == 4354


# ------------------------------------------------------------------ add + RMSNorm prologue

def _bf16(t):
    return t.to(torch.bfloat16)


@pytest.mark.parametrize("which", ["torch", "c"])
def test_rms_norm_closed_form_constant_row(which):
    """x = 2, y = 0, eps = 0: mean(xout²) = 4 exactly, rstd = 0.5, xout·rstd = 1,
    so n must equal w_norm bit for bit (a dropped /K or a wrong sqrt fails)."""
    K = 2560
    x = torch.full((3, K), 2.0, dtype=torch.bfloat16)
    y = torch.zeros((3, K), dtype=torch.bfloat16)
    wn = R.randn_bf16((K,), 321)
    xo, n = (R.add_rms_norm_bf16(x, y, wn, 0.0) if which == "torch" else R.c_add_rms_norm(x, y, wn, 0.0)[:2])
    assert torch.equal(xo, x)
    assert torch.equal(n, wn.expand(3, K))


def test_rms_norm_cancelling_branch_gives_zero():
    x = R.randn_bf16((2, 512), 11)
    xo, n = R.add_rms_norm_bf16(x, -x, R.randn_bf16((512,), 12), 1e-6)
    assert torch.equal(xo.float(), torch.zeros(2, 512)) and torch.equal(n.float(), torch.zeros(2, 512))


def test_rms_norm_torch_and_c_restatements_agree():
    """xout bit-exact; n identical except where the fp32 vs fp64 sum of squares
    moves rstd by an ulp, and then by at most one bf16 ulp."""
    M, K = 5, 2560
    x, y, wn = R.randn_bf16((M, K), 31), R.randn_bf16((M, K), 32, 0.5), R.randn_bf16((K,), 33)
    xo_t, n_t = R.add_rms_norm_bf16(x, y, wn, 1e-6)
    xo_c, n_c, _ = R.c_add_rms_norm(x, y, wn, 1e-6)
    assert torch.equal(xo_t, xo_c)
    bt, bc = R.to_bits(n_t).astype(np.int32), R.to_bits(n_c).astype(np.int32)
    assert np.abs(bt - bc).max() <= 1
    assert (bt == bc).mean() > 0.999


def test_rms_norm_rounds_before_the_gain():
    """The normalised value is rounded to bf16 before the gain multiply
    (engine/kernels/rmsnorm.py:34-43); rounding once at the end is a different
    function and must be told apart on random data."""
    M, K = 4, 2560
    x, y, wn = R.randn_bf16((M, K), 41), R.randn_bf16((M, K), 42), R.randn_bf16((K,), 43)
    xo, n = R.add_rms_norm_bf16(x, y, wn, 1e-6)
    sf = xo.float()
    rstd = torch.rsqrt((sf * sf).mean(-1, keepdim=True) + 1e-6)
    once = (sf * rstd * wn.float()).to(torch.bfloat16)
    assert not torch.equal(once, n)
    twice = ((sf * rstd).to(torch.bfloat16).float() * wn.float()).to(torch.bfloat16)
    assert torch.equal(twice, n)


def test_rms_norm_scale_invariance():
    """With eps = 0, scaling x and y by a power of two scales xout exactly and
    leaves n unchanged."""
    M, K = 3, 1024
    x, y, wn = R.randn_bf16((M, K), 51), R.randn_bf16((M, K), 52), R.randn_bf16((K,), 53)
    xo1, n1 = R.add_rms_norm_bf16(x, y, wn, 0.0)
    xo4, n4 = R.add_rms_norm_bf16(_bf16(x.float() * 4), _bf16(y.float() * 4), wn, 0.0)
    assert torch.equal(xo4.float(), xo1.float() * 4)
    bits1, bits4 = R.to_bits(n1).astype(np.int32), R.to_bits(n4).astype(np.int32)
    assert np.abs(bits1 - bits4).max() <= 1 and (bits1 == bits4).mean() > 0.999


def test_normed_linear_composes_prologue_and_projection():
    M, K, N = 2, 256, 40
    x, y, wn, w = R.randn_bf16((M, K), 61), R.randn_bf16((M, K), 62), R.randn_bf16((K,), 63), R.randn_bf16((N, K), 64, 0.02)
    xo, out = R.normed_linear_bf16(x, y, wn, 1e-6, w)
    assert torch.equal(out, R.linear_bf16(R.add_rms_norm_bf16(x, y, wn, 1e-6)[1], w))
    xo2, out2 = R.normed_gateup_bf16(x, y, wn, 1e-6, R.randn_bf16((2 * N, K), 65, 0.02))
    assert torch.equal(xo, xo2) and out2.shape == (M, N)


# ------------------------------------------------------------------ token selection

def test_topk_rows_k1_is_torch_argmax_and_the_c_restatement():
    logits = R.randn_bf16((6, 3000), 71)
    logits[2, 17] = logits[2].max()        # a tie with an earlier maximum... or a new one
    logits[3, :] = 1.0                     # all equal: index 0
    logits[4, 5] = float("-0.0")
    logits[4, :5] = 0.0                    # -0 ties +0 when 0 is the max
    logits[4, 6:] = -1.0
    idx, _ = R.topk_rows(logits, 1)
    assert torch.equal(idx[:, 0], torch.argmax(logits.float(), dim=-1))
    assert torch.equal(idx[:, 0], R.c_argmax_rows(logits))
    assert idx[3, 0] == 0 and idx[4, 0] == 0


def test_topk_rows_nan_is_the_largest_value():
    logits = R.randn_bf16((2, 50), 72)
    logits[0, 30] = float("nan")
    logits[0, 40] = float("nan")
    logits[1, 7] = float("inf")
    idx, _ = R.topk_rows(logits, 2)
    assert idx[0].tolist() == [30, 40]
    assert idx[0, 0] == torch.argmax(logits.float(), dim=-1)[0]
    assert idx[1, 0] == 7


def test_topk_rows_matches_torch_topk_on_distinct_values():
    g = torch.Generator().manual_seed(73)
    for N in (8, 200, 256):
        vals = torch.randperm(N, generator=g).float().sub_(N // 2)  # distinct integers in [-128, 128): exact in bf16
        logits = vals.reshape(1, N).to(torch.bfloat16)
        for k in (1, 3, 8):
            idx, v = R.topk_rows(logits, k)
            ref = torch.topk(logits.float(), k, dim=-1)
            assert torch.equal(idx, ref.indices) and torch.equal(v.float(), ref.values)


def test_topk_rows_equal_values_take_the_lower_index_first():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0, -5.0]], dtype=torch.bfloat16)
    idx, v = R.topk_rows(logits, 5)
    assert idx[0].tolist() == [1, 2, 4, 3, 0]
    assert v[0].float().tolist() == [3.0, 3.0, 3.0, 2.0, 1.0]
