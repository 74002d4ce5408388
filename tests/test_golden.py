"""Committed fixtures (tests/golden/*.npz, written by make_golden.py) against
the oracle and against the fp64 brute force that pins them."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import gemm_ref as R

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cases(fname):
    data = np.load(GOLDEN / fname)
    names = sorted({k.split("/")[0] for k in data.files})
    return data, names


LIN, LIN_NAMES = _cases("linear_cases.npz")
GU, GU_NAMES = _cases("gateup_cases.npz")


@pytest.mark.parametrize("name", LIN_NAMES)
def test_linear_fixture_is_pinned_by_fp64(name):
    x, w, y = LIN[f"{name}/x"], LIN[f"{name}/w"], LIN[f"{name}/y"]
    exact, mag = R.linear_exact(x, w)
    assert R.within_fp32_bound(R.from_bits(y), exact, mag, x.shape[1]).all()
    assert np.array_equal(LIN[f"{name}/y_exact"], R.f64_to_bf16_bits(exact))


@pytest.mark.parametrize("name", LIN_NAMES)
def test_oracle_reproduces_linear_fixture(name):
    x, w, y = (R.from_bits(LIN[f"{name}/{k}"]) for k in ("x", "w", "y"))
    got = R.linear_bf16(x, w)
    # Same library on another CPU may pick another fp32 order: allow rare
    # one-ulp moves, nothing more.
    diff = R.to_bits(got) != R.to_bits(y)
    assert diff.mean() <= 0.01
    assert R.close(got, y, atol=0, rtol=2 ** -7).all()
    c = R.c_linear_f32(x, w)
    assert R.close(c, y, atol=0, rtol=2 ** -7).all()


@pytest.mark.parametrize("name", GU_NAMES)
def test_gateup_fixture(name):
    x, w, gu, y = (R.from_bits(GU[f"{name}/{k}"]) for k in ("x", "w", "gu", "y"))
    exact, mag = R.linear_exact(x, w)
    assert R.within_fp32_bound(gu, exact, mag, x.shape[1]).all()
    # the epilogue of the fixture's own projection is reproduced exactly
    assert np.array_equal(R.to_bits(R.swiglu_bf16(gu)), R.to_bits(y))
    assert (R.to_bits(R.c_swiglu(gu)) == R.to_bits(y)).mean() > 0.99
    got = R.gateup_bf16(x, w)
    assert R.close(got, y).all()
