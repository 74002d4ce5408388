"""Write the committed golden fixtures under tests/golden/.

The reference (willzeng274/kernel-rush-kawk) holds no golden vectors or
fixtures for its GEMM path, and its kernels are Triton JIT for NVIDIA GPUs,
so the fixtures are produced here from the oracle's library routine
(torch CPU ``F.linear`` on bf16, the reference's ``a @ w.t()``,
engine/kernels/gemm.py:428) and, for every case, the fp64 brute force that
pins it (tests/test_golden.py re-checks both).

Shapes use the real Qwen3-4B K values (2560, 4096, 9728) with truncated N, so
the files stay small.  Seeds follow oracle.gemm_ref.seed_for-style fixed
integers.  Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import gemm_ref as R  # noqa: E402

#: name -> (M, N, K, x_scale, seed)
LINEAR_CASES = {
    "qkv_m1": (1, 48, 2560, 1.0, 11),
    "o_m4": (4, 32, 4096, 1.0, 12),
    "down_m4": (4, 16, 9728, 0.5, 13),
    "lm_m8": (8, 40, 2560, 1.0, 14),
    "verify_m64": (64, 16, 2560, 1.0, 15),
    "ragged_m3": (3, 17, 40, 1.0, 16),
    "ragged_m33": (33, 24, 136, 1.0, 17),
}

#: name -> (M, I, K, seed)
GATEUP_CASES = {
    "gateup_m8": (8, 24, 2560, 21),
    "gateup_m1": (1, 16, 2560, 22),
}


def linear_case(M, N, K, xs, seed):
    x = R.randn_bf16((M, K), seed, xs)
    w = R.randn_bf16((N, K), seed + 500, 0.02)
    y = R.linear_bf16(x, w)
    exact, _ = R.linear_exact(x, w)
    return {"x": R.to_bits(x), "w": R.to_bits(w), "y": R.to_bits(y), "y_exact": R.f64_to_bf16_bits(exact)}


def gateup_case(M, I, K, seed):
    x = R.randn_bf16((M, K), seed)
    w = R.randn_bf16((2 * I, K), seed + 500, 0.02)
    return {"x": R.to_bits(x), "w": R.to_bits(w), "gu": R.to_bits(R.linear_bf16(x, w)),
            "y": R.to_bits(R.gateup_bf16(x, w))}


def argmax_cases():
    """Rows with constructed exact ties at the maximum: the lowest index must win."""
    rng = np.random.default_rng(31)
    rows = []
    idx = []
    for n, ties in ((16, (3, 9)), (1000, (0, 999)), (151936, (70000, 70001, 151935)), (64, (5,))):
        v = rng.standard_normal(n).astype(np.float32)
        top = np.float32(v.max() + 1.0)
        for t in ties:
            v[t] = top
        b = R.f32_to_bf16_bits(v)
        rows.append(b)
        idx.append(min(ties))
    return rows, idx


def main() -> None:
    torch.manual_seed(0)
    out = {}
    for name, (M, N, K, xs, seed) in LINEAR_CASES.items():
        for k, v in linear_case(M, N, K, xs, seed).items():
            out[f"{name}/{k}"] = v
    np.savez_compressed(HERE / "linear_cases.npz", **out)
    out = {}
    for name, (M, I, K, seed) in GATEUP_CASES.items():
        for k, v in gateup_case(M, I, K, seed).items():
            out[f"{name}/{k}"] = v
    np.savez_compressed(HERE / "gateup_cases.npz", **out)
    rows, idx = argmax_cases()
    out = {f"row{i}": r for i, r in enumerate(rows)}
    out["expected"] = np.array(idx, np.int64)
    np.savez_compressed(HERE / "argmax_ties.npz", **out)
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")


if __name__ == "__main__":
    main()
