"""Skinny decode GEMM for Qwen3-4B on MI355X: ``C[M, N] = A[M, K] @ W[N, K]^T``.

Python surface of libkrk_gemm.so, shaped like the reference's
``engine/kernels/gemm.py`` so an engine can swap it in unchanged:

* :class:`SkinnyMatmul` — ``f(a, w) -> a @ w.T`` as a new bf16 tensor
  (reference ``SkinnyMatmul``, engine/kernels/gemm.py:332-361);
* :class:`SkinnyGateUp` — ``f(a, wgu) -> silu(a @ Wg.T) * (a @ Wu.T)`` over the
  concatenated gate-then-up weight (reference ``SkinnyGateUp``,
  engine/kernels/gemm.py:298-329, plus ``swiglu``, engine/kernels/swiglu.py);
* :func:`pick_matmul` / :func:`pick_gateup` — per-shape callables tuned at
  warm-up over the library's candidate configurations and validated against
  ``torch.nn.functional.linear`` on the same device (reference pickers,
  engine/kernels/gemm.py:417-498; search and cache in :mod:`kernels.tune`);
* ``norm=(y, w_norm, xout, eps)`` on every call, :func:`pick_normed` and
  :func:`add_rms_norm` — the residual-add + RMSNorm prologue (reference
  engine/kernels/gemm.py:21-51, 501-560 and engine/kernels/add_rmsnorm.py);
* :class:`SkinnySelect` — the lm_head projection with per-row argmax / top-k
  fused (reference consumers engine/engine.py:196, engine/recycle.py:170);
* :func:`_time` — CUDA/HIP-graph replay timer (engine/kernels/gemm.py:378-414).

All compute runs in the HIP kernels of libkrk_gemm.so; nothing here falls
back to another GEMM.  Calls launch on torch's current stream, allocate only
their output tensor, never synchronise, and may be captured in a graph.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _lib, timing
from ._lib import EPILOGUE_NONE, EPILOGUE_SILU_MUL, GemmConfig

__all__ = [
    "SkinnyMatmul", "SkinnyGateUp", "Gemv", "SkinnySelect", "pick_matmul", "pick_gateup", "pick_normed",
    "add_rms_norm", "gemm_noalloc", "plan", "normed_plan", "resolve", "config_from_triton", "select_plan", "select_fused", "gemm_into", "normed_fused", "tune_projection", "_time",
]


def plan(M: int, N: int, K: int, epilogue: int = EPILOGUE_NONE) -> dict:
    """The configuration the library's dispatch table uses for this shape."""
    cfg = GemmConfig()
    _lib.check(_lib.load().krk_gemm_plan(M, N, K, epilogue, ctypes.byref(cfg)))
    return cfg.as_dict()


def normed_plan(M: int, N: int, K: int, epilogue: int = EPILOGUE_NONE) -> dict:
    """The configuration a normed call of this shape uses without one (fused
    where that measured fastest, else the plain plan behind the prologue
    kernel, ``prologue = 1``)."""
    cfg = GemmConfig()
    _lib.check(_lib.load().krk_gemm_normed_plan(M, N, K, epilogue, ctypes.byref(cfg)))
    return cfg.as_dict()


def _check_operand(name: str, t: torch.Tensor, rows: int | None, cols: int) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if rows is not None and t.shape[0] != rows:
        raise ValueError(f"{name} must have {rows} rows, got shape {tuple(t.shape)}")
    if t.shape[1] != cols:
        raise ValueError(f"{name} must have {cols} columns, got shape {tuple(t.shape)}")
    if t.stride(1) != 1:
        raise ValueError(f"{name} rows must be contiguous (stride(1) == 1), got strides {t.stride()}")


def _check_norm(norm, M: int, K: int, device):
    """Unpack and check ``norm=(y, w_norm, xout, eps)`` (the reference's
    tuple, engine/kernels/gemm.py:346-350)."""
    try:
        d, wn, xout, eps = norm
    except (TypeError, ValueError):
        raise ValueError("norm must be a tuple (y, w_norm, xout, eps)") from None
    _check_operand("norm y", d, M, K)
    _check_operand("xout", xout, M, K)
    if not isinstance(wn, torch.Tensor) or wn.dtype != torch.bfloat16 or wn.numel() != K or not wn.is_contiguous():
        raise ValueError(f"w_norm must be a contiguous bf16 tensor of {K} elements")
    for name, t in (("norm y", d), ("w_norm", wn), ("xout", xout)):
        if t.device != device:
            raise ValueError(f"{name} must be on the operands' device {device}, got {t.device}")
    return d, wn, xout, float(eps)


def gemm_into(x: torch.Tensor, w: torch.Tensor, y: torch.Tensor, epilogue: int = EPILOGUE_NONE,
              workspace: torch.Tensor | None = None, config: dict | None = None, norm=None) -> torch.Tensor:
    """Allocation-free call: ``y = epilogue(x @ w.T)`` into the caller's ``y``.

    Counterpart of the reference's caller-owned-output launcher
    (``launch_gateup64``, engine/kernels/gateup64.py:59-81).  ``workspace`` must
    hold at least ``workspace_bytes`` bytes of zero-filled device memory when
    the plan splits K.  ``norm=(y, w_norm, xout, eps)`` fuses
    ``xout = x + y; x = rms_norm(xout, w_norm)`` in front, as the reference's
    ``norm`` argument does (engine/kernels/gemm.py:346-361).
    """
    M, K = x.shape
    N = w.shape[0]
    _check_operand("x", x, None, K)
    _check_operand("w", w, None, K)
    nout = N // 2 if epilogue == EPILOGUE_SILU_MUL else N
    _check_operand("y", y, M, nout)
    for name, t in (("x", x), ("w", w), ("y", y)):
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be a GPU tensor, got device {t.device}")
    if not (x.device == w.device == y.device):
        raise ValueError(f"operands on different devices: {x.device}, {w.device}, {y.device}")
    if norm is not None:
        d, wn, xout, eps = _check_norm(norm, M, K, x.device)
    ws_ptr, ws_bytes = 0, 0
    if workspace is not None:
        if workspace.device != x.device:
            raise ValueError("workspace must be on the operands' device")
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    lib = _lib.load()
    cfg = GemmConfig.from_dict(config) if config is not None else None
    with torch.cuda.device(x.device):
        if norm is not None:
            head = (x.data_ptr(), x.stride(0), d.data_ptr(), d.stride(0), wn.data_ptr(), eps, xout.data_ptr(),
                    xout.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(), y.stride(0), M, N, K, epilogue)
            if cfg is None:
                rc = lib.krk_gemm_bf16_normed(*head, ws_ptr, ws_bytes, stream)
            else:
                rc = lib.krk_gemm_bf16_normed_config(*head, ctypes.byref(cfg), ws_ptr, ws_bytes, stream)
        elif cfg is None:
            rc = lib.krk_gemm_bf16(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(), y.stride(0),
                                   M, N, K, epilogue, ws_ptr, ws_bytes, stream)
        else:
            rc = lib.krk_gemm_bf16_config(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(),
                                          y.stride(0), M, N, K, epilogue, ctypes.byref(cfg), ws_ptr, ws_bytes, stream)
    _lib.check(rc)
    return y


def gemm_noalloc(x: torch.Tensor, w: torch.Tensor, y: torch.Tensor, epilogue: int = EPILOGUE_NONE) -> torch.Tensor:
    """``y = epilogue(x @ w.T)`` through ``krk_gemm_bf16_noalloc``: no
    workspace argument and no allocation of any kind, for callers that cannot
    allocate (code under graph capture, tight serving loops).  Split-K plans
    use the library's static per-GPU scratch (``KRK_NOALLOC_SCRATCH_BYTES``);
    a plan that does not fit raises ValueError.  Calls that may overlap in
    time on one GPU share that scratch and must not be issued."""
    M, K = x.shape
    N = w.shape[0]
    _check_operand("x", x, None, K)
    _check_operand("w", w, None, K)
    _check_operand("y", y, M, N // 2 if epilogue == EPILOGUE_SILU_MUL else N)
    if not (x.device == w.device == y.device) or x.device.type != "cuda":
        raise ValueError(f"operands must be on one GPU, got {x.device}, {w.device}, {y.device}")
    with torch.cuda.device(x.device):
        rc = _lib.load().krk_gemm_bf16_noalloc(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(),
                                               y.stride(0), M, N, K, epilogue,
                                               torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc)
    return y


def workspace_bytes(M: int, N: int, K: int, epilogue: int = EPILOGUE_NONE, config: dict | None = None,
                    normed: bool = False) -> int:
    lib = _lib.load()
    if normed:
        cfg = GemmConfig.from_dict(config) if config is not None else None
        return int(lib.krk_gemm_normed_workspace_bytes(M, N, K, epilogue, ctypes.byref(cfg) if cfg else None))
    if config is None:
        return int(lib.krk_gemm_workspace_bytes(M, N, K, epilogue))
    cfg = GemmConfig.from_dict(config)
    return int(lib.krk_gemm_config_workspace_bytes(M, N, K, epilogue, ctypes.byref(cfg)))


def normed_fused(M: int, N: int, K: int, epilogue: int = EPILOGUE_NONE, config: dict | None = None) -> bool:
    """Whether a normed call of this shape runs the prologue inside the
    projection kernel (one launch) rather than as a separate kernel."""
    cfg = GemmConfig.from_dict(config) if config is not None else None
    rc = _lib.load().krk_gemm_normed_fused(M, N, K, epilogue, ctypes.byref(cfg) if cfg else None)
    if rc < 0:
        _lib.check(rc)
    return rc == 1


def add_rms_norm(x: torch.Tensor, y: torch.Tensor, weight: torch.Tensor, eps: float,
                 xout: torch.Tensor | None = None) -> torch.Tensor:
    """``xout = x + y`` (bf16; in place into ``x`` when ``xout`` is None) and
    return ``rms_norm(xout, weight)`` — the reference's stand-alone kernel
    (engine/kernels/add_rmsnorm.py:32-43), on libkrk_gemm.so."""
    M, K = x.shape
    _check_operand("x", x, None, K)
    xo = x if xout is None else xout
    d, wn, xo, eps = _check_norm((y, weight, xo, eps), M, K, x.device)
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    with torch.cuda.device(x.device):
        rc = _lib.load().krk_add_rms_norm_bf16(x.data_ptr(), x.stride(0), d.data_ptr(), d.stride(0), wn.data_ptr(),
                                               eps, xo.data_ptr(), xo.stride(0), out.data_ptr(), out.stride(0), M, K,
                                               stream)
    _lib.check(rc)
    return out


_TRITON_KEYS = ("block_n", "block_k", "split_k", "num_warps", "num_stages")


def _largest_at_most(v: int, allowed) -> int:
    fit = [a for a in allowed if a <= v]
    return max(fit) if fit else min(allowed)


def resolve(M: int, N: int, K: int, epilogue: int = EPILOGUE_NONE, config: dict | None = None) -> dict:
    """The configuration the library runs for ``config`` (0 or missing fields
    from the dispatch table); ValueError if this build cannot run it."""
    cfg = GemmConfig.from_dict(config) if config is not None else None
    out = GemmConfig()
    _lib.check(_lib.load().krk_gemm_resolve(M, N, K, epilogue, ctypes.byref(cfg) if cfg else None, ctypes.byref(out)))
    return out.as_dict()


def config_from_triton(M: int, N: int, K: int, epilogue: int, block_n: int, block_k: int, split_k: int,
                       num_warps: int, num_stages: int, persist: int = 0) -> dict:
    """Translate the reference's Triton constructor arguments
    (``SkinnyMatmul / SkinnyGateUp(M, N, K, device, block_n, block_k, split_k,
    num_warps, num_stages, persist)``, ``Gemv(...)``; engine/kernels/gemm.py:251,
    301, 333 and the CONFIGS / GEMV_CONFIGS lists at :284-288, 364-375) into
    the nearest configuration this library instantiates.  The split count and
    the persistent grid carry over; tile sizes map onto the kernel that serves
    the row count:

    * ``persist > 0``: the persistent stream kernel with ``split_k`` K splits,
      raised where needed until each split's K range fits its x registers;
    * at most 8 rows per launch: the VALU kernel with ``num_warps`` waves
      (1, 2, 4 or 8) and ``block_n / num_warps`` W rows per wave (1, 2 or 4);
    * otherwise the LDS-staged MFMA kernel with ``block_n / 16`` W tiles
      (1, 2 or 4), three stages in flight when ``num_stages >= 4``, 512-k
      stages when ``block_k >= 512``.

    SILU_MUL needs an even number of W rows per wave or tile (gate and up).
    Raises ValueError when the library cannot run the result."""
    for name, v in (("block_n", block_n), ("block_k", block_k), ("split_k", split_k), ("num_warps", num_warps),
                    ("num_stages", num_stages)):
        if not isinstance(v, int) or v < 1:
            raise ValueError(f"{name} must be a positive int, got {v!r}")
    silu = epilogue == EPILOGUE_SILU_MUL
    rows = min(M, 64)
    splits = min(split_k, 32)
    if persist:
        cfg = {"kernel": _lib.KERNEL_STREAM, "splits": splits}
    elif rows <= 8:
        waves = _largest_at_most(num_warps, (1, 2, 4, 8))
        per_wave = _largest_at_most(max(1, block_n // waves), (2, 4) if silu else (1, 2, 4))
        cfg = {"kernel": _lib.KERNEL_VALU, "waves": waves, "n_tiles": per_wave,
               "splits": min(splits, -(-K // 512))}
    else:
        tiles = _largest_at_most(max(1, block_n // 16), (2, 4) if silu else (1, 2, 4))
        cfg = {"kernel": _lib.KERNEL_MFMA_LDS, "n_tiles": tiles, "unroll": 3 if num_stages >= 4 else 2,
               "k_chunk": 512 if block_k >= 512 else 256, "splits": splits}
    if persist:
        for sp in range(splits, 33):
            try:
                return resolve(M, N, K, epilogue, dict(cfg, splits=sp))
            except ValueError:
                if sp == 32:
                    raise
    try:
        return resolve(M, N, K, epilogue, cfg)
    except ValueError:
        if cfg.get("unroll") == 3:  # three stages in flight exist only for small tiles
            cfg["unroll"] = 2
            return resolve(M, N, K, epilogue, cfg)
        raise


def _constructor_config(M, N, K, epilogue, config, triton_args: dict, persist: int) -> dict | None:
    given = {k: v for k, v in triton_args.items() if v is not None}
    if not given and not persist:
        return dict(config) if config else None
    if config:
        raise ValueError("give either config= or the reference's Triton arguments, not both")
    missing = [k for k in _TRITON_KEYS if k not in given]
    if missing:
        raise ValueError(f"the reference's constructor arguments come together; missing {', '.join(missing)}")
    return config_from_triton(M, N, K, epilogue, persist=persist, **given)


class SkinnyMatmul:
    """``c = a @ w.T`` for a fixed (M, N, K): bf16 in, fp32 accumulation, bf16 out.

    Mirrors the reference's ``SkinnyMatmul`` (engine/kernels/gemm.py:332-361):
    the split-K workspace belongs to the object and is allocated (zero-filled)
    once here; each call allocates only its output.  It is built like the
    reference's, ``SkinnyMatmul(M, N, K, device, block_n, block_k, split_k,
    num_warps, num_stages, persist=0)`` (the Triton tile arguments are
    translated by :func:`config_from_triton`), or with ``config=`` (keys of
    ``krk_gemm_config``), or with neither (the dispatch table's plan).  A
    configuration this build cannot run raises ValueError here.
    """

    epilogue = EPILOGUE_NONE

    def __init__(self, M: int, N: int, K: int, device, block_n: int | None = None, block_k: int | None = None,
                 split_k: int | None = None, num_warps: int | None = None, num_stages: int | None = None,
                 persist: int = 0, *, config: dict | None = None):
        if M < 1 or N < 1 or K < 8 or K % 8:
            raise ValueError(f"unsupported shape M={M} N={N} K={K} (need K >= 8, K % 8 == 0)")
        self.M, self.N, self.K = M, N, K
        self.device = torch.device(device)
        triton_args = dict(block_n=block_n, block_k=block_k, split_k=split_k, num_warps=num_warps,
                           num_stages=num_stages)
        self.config = _constructor_config(M, N, K, self.epilogue, config, triton_args, persist)
        if self.config is not None:
            resolve(M, N, K, self.epilogue, self.config)  # ValueError now, not at the first call
        # One workspace serves plain and normed calls: both keep their split-K
        # counters at its start; normed calls may use more of it as scratch.
        nbytes = max(workspace_bytes(M, N, K, self.epilogue, self.config),
                     workspace_bytes(M, N, K, self.epilogue, self.config, normed=True))
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=self.device) if nbytes else None
        self.out_cols = N // 2 if self.epilogue == EPILOGUE_SILU_MUL else N

    @property
    def resolved_config(self) -> dict:
        return resolve(self.M, self.N, self.K, self.epilogue, self.config)

    def run(self, a: torch.Tensor, w: torch.Tensor, out: torch.Tensor, norm=None) -> torch.Tensor:
        """Allocation-free form: write into ``out``."""
        if a.shape[0] != self.M or a.shape[1] != self.K or w.shape[0] != self.N:
            raise ValueError(f"operands {tuple(a.shape)} x {tuple(w.shape)} do not match the "
                             f"({self.M}, {self.N}, {self.K}) this object was built for")
        return gemm_into(a, w, out, self.epilogue, self.workspace, self.config, norm)

    def __call__(self, a: torch.Tensor, w: torch.Tensor, norm=None) -> torch.Tensor:
        """``norm=(y, w_norm, xout, eps)`` fuses ``xout = a + y; a = rms_norm(xout, w_norm)``
        in front (reference signature, engine/kernels/gemm.py:346-347)."""
        out = torch.empty((self.M, self.out_cols), dtype=torch.bfloat16, device=a.device)
        return self.run(a, w, out, norm)


class SkinnyGateUp(SkinnyMatmul):
    """``silu(a @ Wg.T) * (a @ Wu.T)`` in one pass over the concatenated weight.

    ``I`` is the intermediate width; the weight is ``[2*I, K]`` with the gate
    rows first (engine/model.py:116).  Rounding follows the reference's three
    bf16 boundaries (engine/kernels/gemm.py:107-113).  Built like the
    reference's ``SkinnyGateUp(M, I, K, device, block_n, block_k, split_k,
    num_warps, num_stages, persist=0)`` (gemm.py:301) or with ``config=``.
    Call as ``f(a, wgu)`` or, like the reference (engine/kernels/gemm.py:314),
    ``f(a, wg, wu)`` with ``wg = wgu[:I]`` and ``wu = wgu[I:]`` views of one
    tensor.
    """

    epilogue = EPILOGUE_SILU_MUL

    def __init__(self, M: int, I: int, K: int, device, block_n: int | None = None, block_k: int | None = None,
                 split_k: int | None = None, num_warps: int | None = None, num_stages: int | None = None,
                 persist: int = 0, *, config: dict | None = None):
        self.I = I
        super().__init__(M, 2 * I, K, device, block_n, block_k, split_k, num_warps, num_stages, persist,
                         config=config)

    def __call__(self, a: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor | None = None, norm=None) -> torch.Tensor:
        wgu = wg if wu is None else _join_halves(wg, wu, self.I)
        return super().__call__(a, wgu, norm)


def _join_halves(wg: torch.Tensor, wu: torch.Tensor, I: int) -> torch.Tensor:
    """The concatenated ``[2I, K]`` view behind ``wg = wgu[:I]``, ``wu = wgu[I:]``."""
    if wg.shape != wu.shape or wg.shape[0] != I or wg.stride() != wu.stride():
        raise ValueError("wg and wu must be the two halves of one [2*I, K] weight")
    gap = (wu.data_ptr() - wg.data_ptr()) // wg.element_size()
    if gap != I * wg.stride(0):
        raise ValueError("wu must start right after wg's I rows (wg = wgu[:I], wu = wgu[I:])")
    return torch.as_strided(wg, (2 * I, wg.shape[1]), wg.stride())


class Gemv(SkinnyMatmul):
    """Row dot products for at most 4 rows (reference ``Gemv``,
    engine/kernels/gemm.py:248-281), built like the reference's ``Gemv(M, N, K,
    device, block_n, block_k, split_k, num_warps, num_stages, gateup=False)``
    or with ``config=``.  ``N`` is the output width; ``gateup=True`` applies
    the SwiGLU epilogue like the reference's GATEUP mode, with the gate and up
    weights passed as ``f(a, wg, wu)`` (halves of one ``[2N, K]`` weight) or
    ``f(a, wgu)``."""

    def __init__(self, M: int, N: int, K: int, device, block_n: int | None = None, block_k: int | None = None,
                 split_k: int | None = None, num_warps: int | None = None, num_stages: int | None = None,
                 gateup: bool = False, *, config: dict | None = None):
        if M > 4:
            raise ValueError("Gemv handles at most 4 rows")
        self.epilogue = EPILOGUE_SILU_MUL if gateup else EPILOGUE_NONE
        self.I = N
        super().__init__(M, 2 * N if gateup else N, K, device, block_n, block_k, split_k, num_warps, num_stages,
                         config=config)

    def __call__(self, a: torch.Tensor, w: torch.Tensor, w2: torch.Tensor | None = None, norm=None) -> torch.Tensor:
        if self.epilogue == EPILOGUE_SILU_MUL and w2 is not None:
            w = _join_halves(w, w2, self.I)
        elif w2 is not None:
            raise ValueError("a second weight is only taken with gateup=True")
        return super().__call__(a, w, norm)


def _time(fn, iters: int = 30, rotate: list | None = None) -> float:
    """Milliseconds per call of ``fn`` (``fn(w)`` over the weights of
    ``rotate`` in turn, else ``fn()``), ``iters`` calls replayed from one
    graph: the reference picker timer's signature
    (engine/kernels/gemm.py:378-414) over :mod:`kernels.timing`."""
    return timing.replay_ms(timing.rotation_calls(fn, iters, rotate))


def _validate(out: torch.Tensor, ref: torch.Tensor, what: str, log=None, silu: bool = False) -> None:
    """The tuner's acceptance (:func:`kernels.tune.close_ok`, ``silu`` for a
    SiLU·mul output): every element within ``2e-2 + 1e-2·|ref|`` and the
    reference's rule (engine/kernels/gemm.py:441-447), max error within
    ``0.02 * max|ref| + 1e-3``.  A failure raises instead of falling back."""
    from . import tune

    ok, why = tune.close_ok(out, ref, silu)
    if not ok:
        raise RuntimeError(f"{what}: HIP GEMM disagrees with F.linear ({why})")
    if log:
        log(f"{what}: validated ({why})")


def _linear_fp32acc(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """torch GEMM with fp32 accumulation forced (the validation reference)."""
    prev = torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    try:
        return F.linear(a, w)
    finally:
        torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = prev


def _silu_mul(gu: torch.Tensor) -> torch.Tensor:
    I = gu.shape[1] // 2
    return F.silu(gu[:, :I]) * gu[:, I:]


def _projection(M: int, N: int, K: int, epilogue: int, device, config: dict | None) -> SkinnyMatmul:
    if epilogue == EPILOGUE_SILU_MUL:
        return SkinnyGateUp(M, N // 2, K, device, config=config)
    return SkinnyMatmul(M, N, K, device, config=config)


def _validation_plan(M: int, epilogue: int, w, rot: list):
    """Weights a tuning candidate is validated on, and whether the
    reference's pointwise M = 64 gate/up rule applies as well.  Every
    candidate runs on the call's weight and a second one of the rotation; a
    gate/up projection of 64 or more rows runs on every distinct weight of the
    rotation and must also meet ``0.02·|ref| + 1e-3`` at every element, as
    the reference's M = 64 gate/up picker requires across its 36 layer
    weights (engine/kernels/m64_gateup_selection.py:71-97)."""
    strict = epilogue == EPILOGUE_SILU_MUL and M >= 64
    if strict:
        checks, seen = [], set()
        for v in [w] + list(rot):
            if id(v) not in seen:
                seen.add(id(v))
                checks.append(v)
    else:
        checks = [w] + [v for v in rot[1:2] if v is not w]
    return checks, strict


def _down_for(checks: list, w, rot: list, down) -> list:
    """The down-projection weight that consumes each checked gate/up weight's
    output: ``down`` is one ``[K_out, I]`` weight, or a list aligned with the
    rotation (layer i's down weight for layer i's gate/up weight; ``w``
    itself pairs with ``down[0]`` when it is not in the rotation)."""
    if down is None:
        return []
    if isinstance(down, torch.Tensor):
        return [down] * len(checks)
    if len(down) != len(rot):
        raise ValueError(f"down: {len(down)} weights for a rotation of {len(rot)}")
    pair = {id(v): d for v, d in zip(rot, down)}
    return [pair.get(id(v), down[0]) for v in checks]


def downstream_ok(out: torch.Tensor, ref: torch.Tensor, wd: torch.Tensor) -> tuple[bool, str]:
    """The consumer check of the reference's N32 gate/up selector
    (engine/kernels/m64_gateup_n32_selection.py:73-105): the candidate's
    gate/up output and the reference's, each run through the same down
    projection (fp32-accumulated torch), must agree under the pointwise
    M = 64 rule."""
    from . import tune

    ok, why = tune.pointwise_ok(_linear_fp32acc(out, wd), _linear_fp32acc(ref, wd))
    return ok, ("down projection: " + why)


def tune_projection(a: torch.Tensor, w: torch.Tensor, epilogue: int = EPILOGUE_NONE, ws: list | None = None,
                    log=None, cache=None, norm=None, limit: int | None = None, down=None):
    """Tune the projection ``a @ w.T`` (with ``epilogue``, and with the
    residual-add + RMSNorm prologue when ``norm=(y, w_norm, eps)``) over the
    library's candidate configurations on this GPU, timing each as a graph
    replay over ``ws``.  Returns a :class:`kernels.tune.Result`; the chosen
    configuration is cached (``cache``, default :func:`kernels.tune.default_cache`).
    ``down``: for a gate/up projection, the down weight(s) that consume its
    output (one tensor, or a list aligned with ``ws``); at 64 rows or more
    each candidate's output must also pass :func:`downstream_ok`."""
    from . import tune

    M, K = a.shape
    N = w.shape[0]
    rot = ws or [w]
    cache = tune.default_cache() if cache is None else cache
    kind = "gateup" if epilogue == EPILOGUE_SILU_MUL else "matmul"
    # Candidates are validated against each weight's own fp32-accumulated
    # torch result (which weights, and which rules: _validation_plan).
    checks, strict = _validation_plan(M, epilogue, w, rot)
    downs = _down_for(checks, w, rot, down) if strict else []

    def judge(out, ref, i=0):
        ok, why = tune.close_ok(out, ref, epilogue == EPILOGUE_SILU_MUL)
        if ok and strict:
            ok, why = tune.pointwise_ok(out, ref)
        if ok and downs:
            ok, why = downstream_ok(out, ref, downs[i])
        return ok, why

    def project(inp, weight):
        ref = _linear_fp32acc(inp, weight)
        return _silu_mul(ref) if epilogue == EPILOGUE_SILU_MUL else ref

    if norm is None:
        refs = [project(a, v) for v in checks]

        def build(cfg):
            mm = _projection(M, N, K, epilogue, a.device, cfg)
            return lambda w_: mm(a, w_)

        def accept(fn):
            for i, (v, ref) in enumerate(zip(checks, refs)):
                ok, why = judge(fn(v), ref, i)
                if not ok:
                    return ok, why
            return ok, why
    else:
        y, w_norm, eps = norm
        kind = "normed-" + kind
        ref_xout, n = _add_rms_norm_ref(a, y, w_norm, eps)
        refs = [project(n, v) for v in checks]
        xout = torch.empty_like(a)

        def build(cfg):
            mm = _projection(M, N, K, epilogue, a.device, cfg)
            return lambda w_: mm(a, w_, norm=(y, w_norm, xout, eps))

        def accept(fn):
            for i, (v, ref) in enumerate(zip(checks, refs)):
                xout.fill_(0)
                out = fn(v)
                if not torch.equal(xout, ref_xout):
                    return False, "xout differs from x + y"
                ok, why = judge(out, ref, i)
                if not ok:
                    return ok, why
            return ok, why
    extra = []
    if norm is not None:
        # A configuration that fuses the prologue into the projection is also
        # timed behind the separate prologue kernel (prologue = 1); both are
        # whole normed calls, like every candidate.
        for cfg in tune.candidates(M, N, K, epilogue):
            if normed_fused(M, N, K, epilogue, cfg):
                extra.append(dict(cfg, prologue=1))
    timer = lambda fn, rot_: _time(fn, rotate=rot_)
    return tune.search(kind, M, N, K, epilogue, a.device, build, accept, timer, rot, log=log, cache=cache, limit=limit,
                       extra=extra, plan=normed_plan(M, N, K, epilogue) if norm is not None else None)


def pick_matmul(a: torch.Tensor, w: torch.Tensor, log=None, ws: list | None = None, tune: bool = True, cache=None):
    """Return ``f(a, w) -> a @ w.T`` for this exact shape (reference
    engine/kernels/gemm.py:417-458).  With ``tune`` the configuration is the
    fastest validated candidate on this GPU (:func:`tune_projection`, within
    the shared :mod:`kernels.budget`), else the dispatch table's.  The chosen
    kernel is validated against ``F.linear`` on the same inputs; with ``log``
    its graph-replay time over the ``ws`` rotation is reported."""
    M, K = a.shape
    N = w.shape[0]
    cfg = tune_projection(a, w, EPILOGUE_NONE, ws, log, cache).config if tune else None
    mm = SkinnyMatmul(M, N, K, a.device, config=cfg)
    _validate(mm(a, w), _linear_fp32acc(a, w), f"matmul M={M} N={N} K={K}", log)
    if log:
        ms = _time(lambda w_: mm(a, w_), rotate=ws or [w])
        log(f"matmul M={M} N={N} K={K}: krk{mm.resolved_config} {ms * 1000:.1f}us "
            f"({2 * M * N * K / ms / 1e6:.0f} GFLOP/s, {N * K * 2 / ms / 1e6:.0f} GB/s)")
    return mm


def pick_gateup(a: torch.Tensor, wgu: torch.Tensor, log=None, ws: list | None = None, tune: bool = True, cache=None,
                down=None):
    """Return ``f(a, wgu) -> silu(a @ Wg.T) * (a @ Wu.T)`` (reference
    engine/kernels/gemm.py:461-498), tuned like :func:`pick_matmul` and
    validated against ``swiglu(F.linear)``.  ``down``: the down weight(s)
    consuming the output (see :func:`tune_projection`)."""
    M, K = a.shape
    I = wgu.shape[0] // 2
    cfg = tune_projection(a, wgu, EPILOGUE_SILU_MUL, ws, log, cache, down=down).config if tune else None
    mm = SkinnyGateUp(M, I, K, a.device, config=cfg)
    _validate(mm(a, wgu), _silu_mul(_linear_fp32acc(a, wgu)), f"gateup M={M} I={I} K={K}", log, silu=True)
    if log:
        ms = _time(lambda w_: mm(a, w_), rotate=ws or [wgu])
        log(f"gateup M={M} I={I} K={K}: krk{mm.resolved_config} {ms * 1000:.1f}us "
            f"({2 * I * K * 2 / ms / 1e6:.0f} GB/s)")
    return mm


def _add_rms_norm_ref(x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, eps: float):
    """Torch composition of the prologue (validation reference): the
    reference's rounding points (engine/kernels/add_rmsnorm.py:20-29)."""
    s = (x.float() + y.float()).to(torch.bfloat16)
    sf = s.float()
    rstd = torch.rsqrt((sf * sf).mean(dim=-1, keepdim=True) + eps)
    return s, ((sf * rstd).to(torch.bfloat16).float() * w_norm.float()).to(torch.bfloat16)


def pick_normed(kind: str, x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, w: torch.Tensor, eps: float,
                log=None, ws: list | None = None, tune: bool = True, cache=None, down=None):
    """Return ``f(x, y, w_norm, xout, w) -> proj(rms_norm(x + y))`` that also
    writes ``xout = x + y`` (reference engine/kernels/gemm.py:501-560).
    ``kind`` is "matmul" or "gateup".  Tuned like :func:`pick_matmul` over
    whole normed calls (the prologue fused or as its own kernel, as each
    configuration runs it), then validated once against the torch
    composition (xout bit-exact, projection under :func:`_validate`'s rule);
    with ``log`` the graph-replay time is logged.  Without tuning the
    library's normed plan runs.  ``down`` (gate/up only): the down weight(s)
    consuming the output, checked at 64 rows or more (:func:`tune_projection`)."""
    if kind not in ("matmul", "gateup"):
        raise ValueError(f"kind must be 'matmul' or 'gateup', got {kind!r}")
    M, K = x.shape
    N = w.shape[0]
    epi = EPILOGUE_SILU_MUL if kind == "gateup" else EPILOGUE_NONE
    cfg = tune_projection(x, w, epi, ws, log, cache, norm=(y, w_norm, eps),
                          down=down if kind == "gateup" else None).config if tune else None
    mm = _projection(M, N, K, epi, x.device, cfg)
    fn = lambda x_, y_, wn_, xout_, w_: mm(x_, w_, norm=(y_, wn_, xout_, eps))
    xout = torch.empty_like(x)
    out = fn(x, y, w_norm, xout, w)
    ref_xout, n = _add_rms_norm_ref(x, y, w_norm, eps)
    ref = _linear_fp32acc(n, w)
    if kind == "gateup":
        ref = _silu_mul(ref)
    if not torch.equal(xout, ref_xout):
        raise RuntimeError(f"normed {kind} M={M} N={N} K={K}: xout differs from x + y")
    _validate(out, ref, f"normed {kind} M={M} N={N} K={K}", log, silu=kind == "gateup")
    if log:
        ms = _time(lambda w_: fn(x, y, w_norm, xout, w_), rotate=ws or [w])
        fused = "fused" if normed_fused(M, N, K, mm.epilogue, cfg) else "prologue kernel"
        log(f"normed {kind} M={M} N={N} K={K}: krk{mm.resolved_config} ({fused}) {ms * 1000:.1f}us")
    return fn


def select_plan(M: int, N: int, K: int, k: int = 1) -> dict:
    """The projection configuration a selecting lm_head call uses for this
    shape and k."""
    cfg = GemmConfig()
    _lib.check(_lib.load().krk_gemm_select_plan(M, N, K, k, ctypes.byref(cfg)))
    return cfg.as_dict()


def select_fused(M: int, N: int, K: int, k: int = 1, config: dict | None = None) -> bool:
    """Whether the selection runs in the projection's epilogue (argmax behind
    a VALU, LDS-staged MFMA or stream projection, top-k behind a stream
    projection of up to 16 rows: the logits are then not written
    unless asked for) rather than in a kernel that reads the logits back."""
    cfg = GemmConfig.from_dict(config) if config else None
    rc = _lib.load().krk_gemm_select_fused(M, N, K, k, ctypes.byref(cfg) if cfg else None)
    _lib.check(min(rc, 0))
    return rc == 1


class SkinnySelect:
    """The lm_head projection followed by token selection: ``f(a, w)`` returns
    the ``[M, k]`` int64 indices of each row's k largest bf16 logits of
    ``a @ w.T`` (largest first, equal values at the lower index first, NaN
    above everything).  ``k = 1`` is ``(a @ w.T).argmax(dim=-1, keepdim=True)``
    (engine/engine.py:196), ``k = 8`` the ``torch.topk(logits, 8).indices`` of
    engine/recycle.py:170.  Argmax behind the VALU, LDS-staged MFMA and stream
    plans, and top-k behind stream plans of up to 16 rows, run in the
    projection's epilogue (``fused``) and write no logits unless ``logits``
    is given; other plans write the logits and select from them.
    ``config`` is the projection's configuration (any plain-epilogue one).
    The workspace belongs to the object (zero-filled once; calls leave it so)."""

    def __init__(self, M: int, N: int, K: int, device, k: int = 1, config: dict | None = None):
        if M < 1 or N < 1 or K < 8 or K % 8:
            raise ValueError(f"unsupported shape M={M} N={N} K={K} (need K >= 8, K % 8 == 0)")
        self.M, self.N, self.K, self.k = M, N, K, k
        self.device = torch.device(device)
        self.config = dict(config) if config else None
        cfg = GemmConfig.from_dict(config) if config else None
        nbytes = int(_lib.load().krk_gemm_select_workspace_bytes(M, N, K, k, ctypes.byref(cfg) if cfg else None))
        if nbytes == 0:
            raise ValueError(f"invalid token selection M={M} N={N} K={K} k={k} config={config}: "
                             f"{_lib.last_error() or 'k must be 1..8 and <= N'}")
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)

    @property
    def resolved_config(self) -> dict:
        return dict(self.config) if self.config else select_plan(self.M, self.N, self.K, self.k)

    @property
    def fused(self) -> bool:
        return select_fused(self.M, self.N, self.K, self.k, self.config)

    def run(self, a: torch.Tensor, w: torch.Tensor, idx: torch.Tensor, logits: torch.Tensor | None = None,
            values: torch.Tensor | None = None) -> torch.Tensor:
        """Allocation-free form: indices into ``idx`` ([M, k] int64), optionally
        the logits into ``logits`` ([M, N] bf16) and the selected values into
        ``values`` ([M, k] bf16)."""
        M, K, N, k = self.M, self.K, self.N, self.k
        _check_operand("a", a, M, K)
        _check_operand("w", w, N, K)
        if logits is not None:
            _check_operand("logits", logits, M, N)
        if idx.dtype != torch.int64 or tuple(idx.shape) != (M, k) or not idx.is_contiguous():
            raise ValueError(f"idx must be a contiguous int64 tensor of shape ({M}, {k})")
        if values is not None and (values.dtype != torch.bfloat16 or tuple(values.shape) != (M, k)
                                   or not values.is_contiguous()):
            raise ValueError(f"values must be a contiguous bf16 tensor of shape ({M}, {k})")
        for name, t in (("a", a), ("w", w), ("idx", idx), ("logits", logits), ("values", values)):
            if t is not None and t.device != self.device:
                raise ValueError(f"{name} must be on {self.device}, got {t.device}")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        lib = _lib.load()
        y_ptr, ldy = (logits.data_ptr(), logits.stride(0)) if logits is not None else (0, N)
        v_ptr = values.data_ptr() if values is not None else 0
        head = (a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), y_ptr, ldy, M, N, K, k, idx.data_ptr(), v_ptr)
        ws = (self.workspace.data_ptr(), self.workspace.numel())
        with torch.cuda.device(self.device):
            if self.config is None:
                rc = lib.krk_gemm_bf16_select(*head, *ws, stream)
            else:
                cfg = GemmConfig.from_dict(self.config)
                rc = lib.krk_gemm_bf16_select_config(*head, ctypes.byref(cfg), *ws, stream)
        _lib.check(rc)
        return idx

    def __call__(self, a: torch.Tensor, w: torch.Tensor, logits: torch.Tensor | None = None) -> torch.Tensor:
        idx = torch.empty((self.M, self.k), dtype=torch.int64, device=a.device)
        return self.run(a, w, idx, logits)
