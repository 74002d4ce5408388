"""Warm-up autotuning of the projection GEMM.

The reference picks, at warm-up and per exact shape, the fastest of cuBLAS
and a list of Triton configurations, each validated against cuBLAS and timed
as a graph replay over every layer's copy of the weight
(engine/kernels/gemm.py:378-414 ``_time``, 417-458 ``pick_matmul``, 461-498
``pick_gateup``, 501-560 ``pick_normed``), within a shared time budget
(engine/budget.py).  Here:

* the search space is the library's own: ``krk_gemm_candidates`` (C ABI)
  lists every configuration it accepts for the shape from a fixed grid, the
  dispatch table's choice first, so the table's plan is always the incumbent;
* a candidate is accepted (:func:`close_ok`) when, on two weights of the
  rotation, every output element is within ``2e-2 + 1e-2 * |ref|`` of an
  fp32-accumulated torch GEMM (a SiLU·mul output's also within the
  reference's gate/up rule ``0.02 * |ref| + 1e-3``) and the reference's own rule, max error within
  ``0.02 * max|ref| + 1e-3`` (gemm.py:441-447), holds too; for normed
  projections xout must also equal x + y bit for bit (gemm.py:548).  A
  rejected candidate is logged and skipped (it would be a kernel bug: every
  configuration computes the same function);
* timing is :func:`kernels.timing.replay_ms` (graph replay, median of 5,
  rotating weights);
* the plan stays unless a challenger beats it by the reference's M = 64
  margin: the fastest few candidates of the sweep are timed again against
  the plan in both orders (plan first, then challenger first), and one
  replaces the plan only if both ratios are below ``MARGIN`` = 0.97
  (engine/kernels/m64_gateup_selection.py:100-128); the challenger with the
  lowest worst ratio wins;
* results go to a ``TuneCache`` keyed by GPU architecture, library build,
  kind and shape, optionally persisted as JSON (``KRK_TUNE_CACHE``), so a
  serving process tunes once per shape and later processes with the same
  library start from the file.

The winner is always a HIP configuration: torch is not a candidate, so a
tuned call never leaves the native path.  Where the reference keeps cuBLAS
when no candidate validates (engine/kernels/gemm.py:449-452), a search here
whose plan fails validation raises: every configuration computes the same
function, so a failing plan is a library fault, not a slower candidate.

Command line (from the package directory, GPU required)::

    python -m kernels.tune --M 1,4,16,64 --out tuned.json
    python -m kernels.tune --tp 8 --out tuned_tp8.json    # one GPU's 8-way shard
"""

from __future__ import annotations

import ctypes
import json
import os
import threading
from dataclasses import dataclass, field

import torch

from . import _lib, budget


def candidates(M: int, N: int, K: int, epilogue: int = _lib.EPILOGUE_NONE) -> list[dict]:
    """Every configuration the library accepts for this shape, plan first."""
    lib = _lib.load()
    n = lib.krk_gemm_candidates(M, N, K, epilogue, None, 0)
    _lib.check(min(n, 0))
    arr = (_lib.GemmConfig * n)()
    got = lib.krk_gemm_candidates(M, N, K, epilogue, arr, n)
    _lib.check(min(got, 0))
    return [c.as_dict() for c in arr[:min(n, got)]]


class TuneCache:
    """Tuned configurations by (architecture, kind, M, N, K); thread-safe.
    With a path, entries are loaded from and written back to a JSON file
    (written whole to a temporary file, then renamed)."""

    def __init__(self, path: str | None = None):
        self.path = path
        self._lock = threading.Lock()
        self._d: dict[str, dict] = {}
        if path and os.path.exists(path):
            with open(path) as f:
                self._d = json.load(f)

    @staticmethod
    def key(device, kind: str, M: int, N: int, K: int) -> str:
        """GPU architecture, library build (``_lib.library_tag``), kind and shape."""
        arch = torch.cuda.get_device_properties(torch.device(device)).gcnArchName.split(":")[0]
        return f"{arch}/{_lib.library_tag()}/{kind}/M{M}/N{N}/K{K}"

    def get(self, key: str) -> dict | None:
        with self._lock:
            e = self._d.get(key)
            return dict(e["config"]) if e else None

    def put(self, key: str, config: dict, us: float) -> None:
        with self._lock:
            self._d[key] = {"config": dict(config), "us": round(us, 2)}
            if self.path:
                tmp = f"{self.path}.tmp{os.getpid()}"
                with open(tmp, "w") as f:
                    json.dump(self._d, f, indent=1, sort_keys=True)
                os.replace(tmp, self.path)

    def entries(self) -> dict:
        with self._lock:
            return json.loads(json.dumps(self._d))


_default_cache: TuneCache | None = None
_default_lock = threading.Lock()


def default_cache() -> TuneCache:
    """The process-wide cache (file from ``KRK_TUNE_CACHE`` when set)."""
    global _default_cache
    with _default_lock:
        if _default_cache is None:
            _default_cache = TuneCache(os.environ.get("KRK_TUNE_CACHE") or None)
        return _default_cache


@dataclass
class Trial:
    config: dict
    us: float | None          # None: rejected or failed
    note: str = ""


@dataclass
class Result:
    config: dict
    us: float
    plan_us: float | None     # the dispatch table's configuration, when measured
    cached: bool = False
    trials: list = field(default_factory=list)
    # (challenger config, ratio with the plan timed first, ratio with the
    # challenger timed first) for every challenger confirmed against the plan
    confirmations: list = field(default_factory=list)


# A challenger replaces the plan only when it takes less than this fraction
# of the plan's time in each of two opposite-order timings
# (engine/kernels/m64_gateup_selection.py:124-128).
MARGIN = 0.97
# Fastest challengers of the sweep that are confirmed against the plan.
CONFIRM = 3


def confirm_ratios(plan_fn, cand_fn, timer, rot) -> tuple[float, float] | None:
    """Challenger / plan time ratios from two opposite-order timings: plan
    then challenger, then challenger then plan (the reference's
    ``candidate_first in (False, True)`` loop, m64_gateup_selection.py:100-120).
    None when a timing is not a positive finite number or the budget ran out
    (the plan is kept)."""
    import math

    ratios = []
    for cand_first in (False, True):
        times = {}
        for which in (("cand", "plan") if cand_first else ("plan", "cand")):
            if budget.expired():
                return None
            ms = timer(cand_fn if which == "cand" else plan_fn, rot)
            if not (isinstance(ms, (int, float)) and math.isfinite(ms) and ms > 0):
                return None
            times[which] = ms
        ratios.append(times["cand"] / times["plan"])
    return ratios[0], ratios[1]


def close_ok(out: torch.Tensor, ref: torch.Tensor, silu: bool = False) -> tuple[bool, str]:
    """Acceptance of one candidate output against the fp32-accumulated torch
    reference.  Two rules, both required:

    * elementwise, the bar this library is held to:
      ``|out - ref| <= 2e-2 + 1e-2 * |ref|`` at every element, with NaN
      exactly where the reference has NaN and infinities equal.  For a
      SiLU·mul output (``silu``) an element may instead meet the reference's
      own gate/up rule ``0.02 * |ref| + 1e-3``
      (engine/kernels/m64_gateup_selection.py:71-97), which is looser for
      ``|ref| > ~1.9``: the three bf16 roundings of the epilogue turn a gate
      or up sum that lands on the other side of a rounding midpoint than
      torch's (the two fp32 summation orders differ) into a few ulps of the
      product.  Seen on an MI355X: gate 2.0078133 (exact), 8e-7 above the
      midpoint of 2 and 2.015625, rounded up by the kernel and down by torch,
      gave 6.719 against 6.625;
    * globally, the reference's own picker rule (engine/kernels/gemm.py:441-447):
      ``max|out - ref| <= 0.02 * max|ref| + 1e-3`` over the finite elements.
    """
    out, ref = out.float(), ref.float()
    if out.shape != ref.shape:
        return False, f"shape {tuple(out.shape)} vs {tuple(ref.shape)}"
    nan_o, nan_r = out.isnan(), ref.isnan()
    if not torch.equal(nan_o, nan_r):
        return False, f"NaN at {int((nan_o != nan_r).sum())} positions where the reference differs"
    inf_r = ref.isinf()
    if not torch.equal(out.isinf(), inf_r) or not torch.equal(out[inf_r], ref[inf_r]):
        return False, "infinities differ from the reference"
    fin = ~(nan_r | inf_r)
    o, r = out[fin], ref[fin]
    if o.numel() == 0:
        return True, "no finite elements"
    err = (o - r).abs()
    bar = 2e-2 + 1e-2 * r.abs()
    if silu:
        bar = torch.maximum(bar, 0.02 * r.abs() + 1e-3)
    bad = int((err > bar).sum())
    if bad:
        rule = "max(2e-2 + 1e-2*|ref|, 0.02*|ref| + 1e-3)" if silu else "2e-2 + 1e-2*|ref|"
        return False, f"{bad} elements outside {rule} (max err {err.max().item():.4g})"
    worst = err.max().item()
    tol = 0.02 * r.abs().max().item() + 1e-3
    if not worst <= tol:
        return False, f"max err {worst:.4g} > reference rule {tol:.4g}"
    return True, f"max err {worst:.4g}"


def pointwise_ok(out: torch.Tensor, ref: torch.Tensor) -> tuple[bool, str]:
    """The reference's acceptance of its M = 64 gate/up kernels
    (engine/kernels/m64_gateup_selection.py:71-97): both outputs finite and
    ``|out - ref| <= 0.02 * |ref| + 1e-3`` at every element (tighter than
    :func:`close_ok`'s elementwise bar wherever ``|ref| < ~1.9``)."""
    out, ref = out.float(), ref.float()
    if out.shape != ref.shape:
        return False, f"shape {tuple(out.shape)} vs {tuple(ref.shape)}"
    if not (torch.isfinite(out).all() and torch.isfinite(ref).all()):
        return False, "non-finite output or reference"
    err = (out - ref).abs()
    bad = int((err > 0.02 * ref.abs() + 1e-3).sum())
    if bad:
        return False, f"{bad} elements outside 0.02*|ref| + 1e-3 (max err {err.max().item():.4g})"
    return True, f"max err {err.max().item():.4g}"


def search(kind: str, M: int, N: int, K: int, epilogue: int, device, build, accept, timer, rot: list,
           log=None, cache: TuneCache | None = None, limit: int | None = None,
           extra: list | None = None, plan: dict | None = None) -> Result:
    """Tune one shape.

    build(cfg) -> fn(w) runs the candidate on weight w and returns its output;
    accept(fn) -> (ok, text) validates one call; timer(fn, rot) -> ms per call.
    The candidates are the library's (:func:`candidates`, led by the plan)
    followed by ``extra``; ``plan`` replaces the library's plan at the head
    (the normed calls' own plan).  The plan (first candidate) is always
    measured; the rest while the budget lasts (at most ``limit`` candidates
    in all when given).  The ``CONFIRM`` fastest candidates that beat the
    plan's sweep time are then timed against it in both orders
    (:func:`confirm_ratios`); the plan is kept unless one of them clears
    ``MARGIN`` in both.  If the plan itself is rejected or cannot be timed,
    the fastest validated candidate is taken as it stands."""
    key = TuneCache.key(device, kind, M, N, K) if cache is not None else None
    if cache is not None:
        hit = cache.get(key)
        if hit is not None:
            if log:
                log(f"tune {kind} M={M} N={N} K={K}: cached krk{hit}")
            return Result(hit, float("nan"), None, cached=True)
    cands = candidates(M, N, K, epilogue) + list(extra or [])
    if plan is not None:
        cands = [plan] + [c for c in cands if c != plan]
    if limit is not None:
        cands = cands[:max(1, limit)]
    trials: list[Trial] = []
    timed: list[tuple[float, int, dict, object]] = []  # (us, sweep index, config, fn)
    plan_us = None
    plan_fn = None
    for i, cfg in enumerate(cands):
        if i > 0 and budget.expired():
            break
        try:
            fn = build(cfg)
            ok, why = accept(fn)
            if not ok:
                trials.append(Trial(cfg, None, "rejected: " + why))
                if log:
                    log(f"tune {kind} M={M} N={N} K={K}: krk{cfg} rejected ({why})")
                continue
            us = timer(fn, rot) * 1000.0
        except (ValueError, RuntimeError) as exc:  # a configuration this shape cannot use
            trials.append(Trial(cfg, None, f"failed: {exc}"))
            continue
        trials.append(Trial(cfg, us))
        if i == 0:
            plan_us, plan_fn = us, fn
        timed.append((us, i, cfg, fn))
    if not timed:
        raise RuntimeError(f"tune {kind} M={M} N={N} K={K}: no candidate passed validation")
    timed.sort(key=lambda t: (t[0], t[1]))
    confirmations = []
    if plan_fn is None:
        # No incumbent to beat: the fastest validated candidate as timed.
        best_us, _, best_cfg, _ = timed[0]
    else:
        best_us, best_cfg, best_ratio = plan_us, cands[0], 1.0
        for us, _, cfg, fn in [t for t in timed if t[1] != 0 and t[0] < plan_us][:CONFIRM]:
            r = confirm_ratios(plan_fn, fn, timer, rot)
            if r is None:
                break
            confirmations.append((cfg, r[0], r[1]))
            worst = max(r)
            if log:
                log(f"tune {kind} M={M} N={N} K={K}: krk{cfg} against the plan {r[0]:.4f} / {r[1]:.4f}")
            if worst < MARGIN and worst < best_ratio:
                best_us, best_cfg, best_ratio = us, cfg, worst
    res = Result(best_cfg, best_us, plan_us, trials=trials, confirmations=confirmations)
    if cache is not None:
        cache.put(key, res.config, res.us)
    if log:
        gain = f", plan {plan_us:.1f}us" if plan_us is not None else ""
        log(f"tune {kind} M={M} N={N} K={K}: krk{res.config} {res.us:.1f}us over {len(trials)} candidates{gain}")
    return res


def _us_text(r: Result) -> str:
    """The CLI's timing column: a cache hit carries no new measurement, and
    the plan may have failed to time."""
    if r.cached:
        return "cached (tuned earlier by this library build)"
    plan = f"{r.plan_us:8.2f} us" if r.plan_us is not None else "       - "
    return f"plan {plan}  tuned {r.us:8.2f} us"


def main(argv=None) -> int:
    import argparse

    from . import gemm as G

    p = argparse.ArgumentParser(description="Tune the Qwen3-4B decode projections on this GPU.")
    p.add_argument("--M", default="1,2,4,8,16,32,64", help="comma-separated row counts")
    p.add_argument("--shapes", default="qkv,o,gate_up,down,lm_head")
    p.add_argument("--copies", type=int, default=8, help="distinct weight copies rotated while timing")
    p.add_argument("--out", default=None, help="JSON cache file to write")
    p.add_argument("--seconds", type=float, default=0.0, help="budget per shape (0: no limit)")
    p.add_argument("--tp", type=int, default=1,
                   help="tune one GPU's shard under this tensor-parallel degree (N of qkv, gate_up and lm_head, "
                        "K of o and down divided by it)")
    args = p.parse_args(argv)
    t = args.tp
    if t < 1 or 6144 % t or 9728 % t or 4096 % t or 151936 % t:
        p.error(f"--tp {t} does not divide the Qwen3-4B shapes")
    shapes = {"qkv": (2560, 6144 // t, 0), "o": (4096 // t, 2560, 0), "gate_up": (2560, 2 * (9728 // t), 1),
              "down": (9728 // t, 2560, 0), "lm_head": (2560, 151936 // t, 0)}
    dev = torch.device("cuda:0")
    cache = TuneCache(args.out)
    g = torch.Generator(device=dev).manual_seed(0)
    rows = []
    for name in args.shapes.split(","):
        K, N, epi = shapes[name]
        copies = max(2, min(args.copies * t, -(-(300 << 20) // (N * K * 2)))) if t > 1 else \
            (2 if name == "lm_head" else args.copies)
        ws = [torch.randn((N, K), device=dev, generator=g).mul_(0.02).to(torch.bfloat16) for _ in range(copies)]
        for M in map(int, args.M.split(",")):
            a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
            if args.seconds > 0:
                budget.start(args.seconds)
            else:
                budget.clear()
            r = G.tune_projection(a, ws[0], epi, ws=ws, cache=cache)
            rows.append((name, M, r.plan_us, r.us, r.config))
            print(f"{name:8s} M={M:3d} {_us_text(r)}  krk{r.config}", flush=True)
            del a
        del ws
        torch.cuda.empty_cache()
    budget.clear()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
