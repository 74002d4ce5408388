"""CPU oracle for the skinny decode GEMM — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker; the product path never imports it.

What it restates (willzeng274/kernel-rush-kawk):

* :func:`linear_bf16` — the projection ``C = A @ W.T`` in bf16 with fp32
  accumulation.  The reference's incumbent for every shape is torch
  ``a @ w.t()`` (engine/kernels/gemm.py:428, engine/model.py:153-158), i.e.
  ``torch.nn.functional.linear`` on bf16 tensors; its Triton kernels accumulate
  in fp32 and round once (gemm.py:90, 240).  This oracle calls that same
  library routine on the CPU.
* :func:`swiglu_bf16` / :func:`gateup_bf16` — SwiGLU over the gate-first
  ``[M, 2I]`` layout with three bf16 roundings (engine/kernels/swiglu.py:14-33,
  gemm.py:107-113; gate/up concatenation order engine/model.py:116).
* :func:`argmax_rows` — lm_head token selection, first index on ties
  (engine/engine.py:196, engine/model.py:365, OPTIMIZATION_GUIDE.md:213).

How each is pinned (tests/test_oracle.py) — the reference ships no golden
vectors or kernel tests for this path (its only test is tests/test_client.py,
an HTTP mock), so the pins are mathematical:

* linear_bf16: fp64 brute force (:func:`linear_exact`) with a rigorous fp32
  summation error bound (:func:`within_fp32_bound`); special cases (x = 0,
  one-hot x selects a column exactly, identity block, negation symmetry,
  non-square shapes that fail under a transposed operand); the independent C
  restatement (gemm_ref.c); committed fixtures tests/golden/*.npz.
* swiglu_bf16: closed form with explicit roundings evaluated in fp64 and by
  the C restatement; a case where one rounding and three roundings differ;
  gate/up order swap detection; special values (0, large ±).
* argmax_rows: constructed ties (lowest index wins), NaN-free random rows
  against the C restatement.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

# --------------------------------------------------------------------------
# torch-CPU restatement (the reference's own library call)
# --------------------------------------------------------------------------


def linear_bf16(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, w)`` on CPU bf16 tensors: fp32 accumulation, bf16 result.
    Reference: engine/kernels/gemm.py:428 (``a @ w.t()``)."""
    return F.linear(x.detach().to("cpu", torch.bfloat16), w.detach().to("cpu", torch.bfloat16))


def swiglu_bf16(gu: torch.Tensor) -> torch.Tensor:
    """``silu(gu[:, :I]) * gu[:, I:]`` on bf16: silu in fp32 rounded to bf16,
    product rounded to bf16.  Reference: engine/kernels/swiglu.py:14-33."""
    gu = gu.detach().to("cpu", torch.bfloat16)
    I = gu.shape[1] // 2
    return F.silu(gu[:, :I]) * gu[:, I:]


def gateup_bf16(x: torch.Tensor, wgu: torch.Tensor) -> torch.Tensor:
    """``swiglu(x @ wgu.T)`` — the reference's cuBLAS+SwiGLU incumbent
    (engine/kernels/gemm.py:469): projection rounds to bf16, then SwiGLU."""
    return swiglu_bf16(linear_bf16(x, wgu))


def add_rms_norm_bf16(x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, eps: float):
    """Residual add + RMSNorm with the reference's rounding points: returns
    ``(xout, n)`` with ``xout = bf16(x + y)`` and
    ``n = bf16(bf16(xout · rsqrt(mean(xout²) + eps)) · w_norm)``, the mean of
    squares accumulated in fp32.  Reference: engine/kernels/add_rmsnorm.py:15-29
    (``add_rms_norm``), engine/kernels/gemm.py:21-51 (``_norm_stats`` and
    ``_normed_tile``, the fused prologue), cast placement per
    engine/kernels/rmsnorm.py:34-43."""
    x = x.detach().to("cpu", torch.bfloat16).float()
    y = y.detach().to("cpu", torch.bfloat16).float()
    wn = w_norm.detach().to("cpu", torch.bfloat16).float()
    s = (x + y).to(torch.bfloat16)
    sf = s.float()
    rstd = torch.rsqrt((sf * sf).sum(dim=-1, keepdim=True) / sf.shape[-1] + eps)
    n = (sf * rstd).to(torch.bfloat16).float() * wn
    return s, n.to(torch.bfloat16)


def normed_linear_bf16(x, y, w_norm, eps, w):
    """``(xout, n @ w.T)``: the pick_normed contract for "matmul"
    (engine/kernels/gemm.py:501-560, engine/model.py:166)."""
    xout, n = add_rms_norm_bf16(x, y, w_norm, eps)
    return xout, linear_bf16(n, w)


def normed_gateup_bf16(x, y, w_norm, eps, wgu):
    """``(xout, swiglu(n @ wgu.T))``: the pick_normed contract for "gateup"."""
    xout, n = add_rms_norm_bf16(x, y, w_norm, eps)
    return xout, gateup_bf16(n, wgu)


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """Per-row index of the maximum, lowest index on ties (torch.argmax
    returns the first occurrence).  Reference: engine/engine.py:196."""
    return torch.argmax(logits.detach().to("cpu").float(), dim=-1)


def topk_rows(logits: torch.Tensor, k: int):
    """Per-row indices and values of the k largest bf16 logits: larger value
    first, equal values at the lower index first, every NaN above +inf, -0
    equal to +0.  k = 1 is torch.argmax's choice (engine/engine.py:196, lowest
    index on ties per OPTIMIZATION_GUIDE.md:213); for distinct values it is
    torch.topk's (engine/recycle.py:170), whose order among equal values is
    unspecified."""
    b = to_bits(logits.detach().to("cpu", torch.bfloat16)).astype(np.uint32)
    nan = (b & 0x7FFF) > 0x7F80
    b = np.where(b == 0x8000, 0, b)
    o = np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000)
    o = np.where(nan, 0xFFFF, o).astype(np.int64)
    M, N = o.shape
    n_idx = np.arange(N, dtype=np.int64)
    key = (o << 32) - n_idx[None, :]          # larger value, then lower index, is larger
    order = np.argsort(-key, axis=1, kind="stable")[:, :k]
    vals = np.take_along_axis(to_bits(logits.detach().to("cpu", torch.bfloat16)), order, axis=1)
    return torch.from_numpy(order), from_bits(vals)


# --------------------------------------------------------------------------
# bf16 bit helpers (numpy has no bf16 dtype; bf16 travels as uint16 bits)
# --------------------------------------------------------------------------


def to_bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 numpy array of its bit patterns."""
    return t.detach().to("cpu", torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray) -> torch.Tensor:
    """uint16 bit patterns -> bf16 CPU tensor."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def bits_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (NaN -> quiet NaN)."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def f64_to_bf16_bits(d: np.ndarray) -> np.ndarray:
    """fp64 -> bf16 bits with a single round-to-nearest-even (no double rounding)."""
    d = np.asarray(d, dtype=np.float64)
    f = d.astype(np.float32)
    u = f.view(np.uint32).astype(np.int64)
    mid = ((u & 0xFFFF) == 0x8000) & (f.astype(np.float64) != d)
    above = np.abs(d) > np.abs(f.astype(np.float64))
    u = np.where(mid, np.where(above, u + 1, u - 1), u)
    return f32_to_bf16_bits(u.astype(np.uint32).view(np.float32))


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (8 significant bits); 2^-133 floor."""
    v = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return np.exp2(e - 7)


# --------------------------------------------------------------------------
# fp64 brute force and error bounds
# --------------------------------------------------------------------------


def linear_exact(x: torch.Tensor | np.ndarray, w: torch.Tensor | np.ndarray):
    """Exact ``x @ w.T`` of bf16 operands in fp64 (each product is exact in
    fp64) and ``|x| @ |w|.T``, the magnitude that bounds summation error."""
    xb = to_bits(x) if isinstance(x, torch.Tensor) else np.asarray(x, np.uint16)
    wb = to_bits(w) if isinstance(w, torch.Tensor) else np.asarray(w, np.uint16)
    xf = bits_to_f32(xb).astype(np.float64)
    wf = bits_to_f32(wb).astype(np.float64)
    return xf @ wf.T, np.abs(xf) @ np.abs(wf).T


def fp32_sum_bound(abssum: np.ndarray, K: int) -> np.ndarray:
    """Worst-case error of any fp32 summation order of K exact products:
    (K-1)·u·Σ|p| with u = 2^-24 (Higham, recursive summation; tree or blocked
    orders have smaller constants), padded by 1% for fp64 evaluation noise."""
    return 1.01 * (K - 1) * 2.0 ** -24 * np.asarray(abssum, np.float64)


def within_fp32_bound(y: torch.Tensor, exact: np.ndarray, abssum: np.ndarray, K: int) -> np.ndarray:
    """Elementwise: is the bf16 result ``y`` a correct rounding of SOME fp32
    sum of the products?  |y - exact| <= E + ulp_bf16(|exact| + E)/2."""
    yf = bits_to_f32(to_bits(y)).astype(np.float64)
    E = fp32_sum_bound(abssum, K)
    return np.abs(yf - exact) <= E + 0.5 * bf16_ulp(np.abs(exact) + E) * (1 + 2.0 ** -20)


def close(out: torch.Tensor, ref: torch.Tensor, atol: float = 2e-2, rtol: float = 1e-2) -> np.ndarray:
    """North-star parity rule: |out - ref| <= atol + rtol·|ref| (elementwise)."""
    o = out.detach().to("cpu").double().numpy()
    r = ref.detach().to("cpu").double().numpy()
    return np.abs(o - r) <= atol + rtol * np.abs(r)


# --------------------------------------------------------------------------
# C restatement (oracle/_build/liboracle.so)
# --------------------------------------------------------------------------

_C = None


def c_lib() -> ctypes.CDLL:
    """Load oracle/_build/liboracle.so, building it with gcc if it is absent."""
    global _C
    if _C is None:
        from . import build as _build
        if not _build.LIB.exists():
            _build.build()
        lib = ctypes.CDLL(str(_build.LIB))
        P = ctypes.c_void_p
        i64, i32 = ctypes.c_int64, ctypes.c_int
        lib.oracle_linear_f32.argtypes = [P, i64, P, i64, P, i64, i32, i32, i32]
        lib.oracle_linear_f64.argtypes = [P, i64, P, i64, P, P, P, i32, i32, i32]
        lib.oracle_silu_mul1.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        lib.oracle_silu_mul1.restype = ctypes.c_uint16
        lib.oracle_swiglu.argtypes = [P, i64, P, i64, i32, i32]
        lib.oracle_gateup_f32.argtypes = [P, i64, P, i64, P, i64, i32, i32, i32]
        lib.oracle_argmax_rows.argtypes = [P, i64, i32, i32, P]
        lib.oracle_add_rms_norm.argtypes = [P, i64, P, i64, P, ctypes.c_double, P, P, i64, i32, i32, P]
        _C = lib
    return _C


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def c_linear_f32(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    xb, wb = to_bits(x), to_bits(w)
    M, K = xb.shape
    N = wb.shape[0]
    y = np.empty((M, N), np.uint16)
    c_lib().oracle_linear_f32(_ptr(xb), K, _ptr(wb), K, _ptr(y), N, M, N, K)
    return from_bits(y)


def c_linear_f64(x: torch.Tensor, w: torch.Tensor):
    """(exact fp64, Σ|p| fp64, singly-rounded bf16 tensor) from the C brute force."""
    xb, wb = to_bits(x), to_bits(w)
    M, K = xb.shape
    N = wb.shape[0]
    ex = np.empty((M, N), np.float64)
    ab = np.empty((M, N), np.float64)
    y = np.empty((M, N), np.uint16)
    c_lib().oracle_linear_f64(_ptr(xb), K, _ptr(wb), K, _ptr(ex), _ptr(ab), _ptr(y), M, N, K)
    return ex, ab, from_bits(y)


def c_swiglu(gu: torch.Tensor) -> torch.Tensor:
    b = to_bits(gu)
    M, two_i = b.shape
    I = two_i // 2
    out = np.empty((M, I), np.uint16)
    c_lib().oracle_swiglu(_ptr(b), two_i, _ptr(out), I, M, I)
    return from_bits(out)


def c_gateup_f32(x: torch.Tensor, wgu: torch.Tensor) -> torch.Tensor:
    xb, wb = to_bits(x), to_bits(wgu)
    M, K = xb.shape
    I = wb.shape[0] // 2
    out = np.empty((M, I), np.uint16)
    c_lib().oracle_gateup_f32(_ptr(xb), K, _ptr(wb), K, _ptr(out), I, M, I, K)
    return from_bits(out)


def c_argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    b = to_bits(logits)
    M, N = b.shape
    idx = np.empty((M,), np.int64)
    c_lib().oracle_argmax_rows(_ptr(b), N, M, N, _ptr(idx))
    return torch.from_numpy(idx)


def c_add_rms_norm(x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, eps: float):
    """(xout, n, rstd fp64) from the C restatement: statistics in fp64, the
    same three bf16 rounding points."""
    xb, yb, wb = to_bits(x), to_bits(y), to_bits(w_norm.reshape(1, -1))
    M, K = xb.shape
    xo = np.empty((M, K), np.uint16)
    n = np.empty((M, K), np.uint16)
    rstd = np.empty((M,), np.float64)
    c_lib().oracle_add_rms_norm(_ptr(xb), K, _ptr(yb), K, _ptr(wb), float(eps), _ptr(xo), _ptr(n), K, M, K, _ptr(rstd))
    return from_bits(xo), from_bits(n), rstd


# --------------------------------------------------------------------------
# Seeded synthetic inputs of the BASELINE configs
# --------------------------------------------------------------------------

HIDDEN, INTER, VOCAB, LAYERS, Q_WIDTH = 2560, 9728, 151936, 36, 4096

#: (name, K, N_w, epilogue) of the five Qwen3-4B projections (engine/model.py:112-116,
#: OPTIMIZATION_GUIDE.md:119-131).
SHAPES = {
    "qkv": (HIDDEN, 6144, "none"),
    "o": (Q_WIDTH, HIDDEN, "none"),
    "gate_up": (HIDDEN, 2 * INTER, "silu_mul"),
    "down": (INTER, HIDDEN, "none"),
    "lm_head": (HIDDEN, VOCAB, "none"),
}

TENSOR_ID = {"x": 0, "qkv": 1, "o": 2, "gate_up": 3, "down": 4, "lm_head": 5}


def seed_for(config: int, layer: int, tensor: str) -> int:
    """Seed scheme: 1000·config + 10·layer + tensor-id."""
    return 1000 * config + 10 * layer + TENSOR_ID[tensor]


def randn_bf16(shape, seed: int, scale: float = 1.0, device="cpu") -> torch.Tensor:
    """N(0, 1)·scale rounded to bf16, from a seeded generator on ``device``."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = torch.randn(shape, generator=g, dtype=torch.float32, device=device)
    if scale != 1.0:
        t.mul_(scale)
    return t.to(torch.bfloat16)
