"""Host logic of the warm-up tuner: the budget clock and the tuned-config
cache (reference engine/budget.py; the cache has no reference counterpart,
it keeps the pickers' results across processes)."""

from __future__ import annotations

import json
import time

from kernels import budget
from kernels.tune import TuneCache


def test_budget_deadline():
    budget.clear()
    assert not budget.expired() and budget.remaining() == float("inf")
    budget.start(0.05)
    assert not budget.expired() and 0 < budget.remaining() <= 0.05
    time.sleep(0.06)
    assert budget.expired() and budget.remaining() < 0
    budget.clear()
    assert not budget.expired()


def test_cache_memory_and_file(tmp_path):
    mem = TuneCache()
    assert mem.get("gfx950/matmul/M1/N6144/K2560") is None
    cfg = {"kernel": 2, "m_tiles": 1, "n_tiles": 1, "unroll": 5, "waves": 8, "splits": 1, "k_chunk": 0}
    mem.put("gfx950/matmul/M1/N6144/K2560", cfg, 6.281)
    got = mem.get("gfx950/matmul/M1/N6144/K2560")
    assert got == cfg and got is not cfg          # a copy: callers cannot edit the cache
    path = tmp_path / "tuned.json"
    disk = TuneCache(str(path))
    disk.put("gfx950/gateup/M32/N19456/K2560", cfg, 24.7)
    disk.put("gfx950/matmul/M1/N6144/K2560", cfg, 6.3)
    data = json.loads(path.read_text())
    assert data["gfx950/gateup/M32/N19456/K2560"] == {"config": cfg, "us": 24.7}
    assert not list(tmp_path.glob("*.tmp*"))      # written whole, then renamed
    again = TuneCache(str(path))
    assert again.get("gfx950/gateup/M32/N19456/K2560") == cfg
    assert set(again.entries()) == set(data)


def test_cache_key_names_the_library_build(monkeypatch):
    """Entries are keyed by architecture, library digest, kind and shape, so a
    rebuilt library never reuses another build's tuned configurations."""
    from kernels import _lib, tune

    class Props:
        gcnArchName = "gfx950:sramecc+:xnack-"

    monkeypatch.setattr(tune.torch.cuda, "get_device_properties", lambda dev: Props())
    tag = _lib.library_tag()
    assert len(tag) == 12 and tag == _lib.library_tag()
    assert TuneCache.key("cuda:0", "matmul", 1, 6144, 2560) == f"gfx950/{tag}/matmul/M1/N6144/K2560"


class _EngineBudget:
    """Stands in for the reference engine's ``budget`` module
    (engine/budget.py: start / expired / remaining over one deadline)."""

    def __init__(self, expired: bool):
        self.is_expired = expired
        self.started = []

    def start(self, seconds):
        self.started.append(seconds)

    def expired(self):
        return self.is_expired

    def remaining(self):
        return -1.0 if self.is_expired else 100.0


def _search_with_stubs(monkeypatch, M=8, N=6144, K=2560):
    """tune.search over the library's real candidate list with a fake build,
    acceptance and timer: returns (result, configs that were timed)."""
    from kernels import tune

    timed = []

    def build(cfg):
        return lambda w: cfg

    def accept(fn):
        return True, "stub"

    def timer(fn, rot):
        cfg = fn(None)
        timed.append(cfg)
        return 1.0 + 0.01 * len(timed)

    res = tune.search("matmul", M, N, K, 0, "cpu", build, accept, timer, [None], cache=None)
    return res, timed


def test_engine_budget_module_is_the_pickers_clock(monkeypatch):
    """With the engine's ``budget`` module loaded and its deadline passed,
    the tuner measures the dispatch table's plan and nothing else."""
    import sys

    from kernels import budget, tune

    budget.use(None)
    engine = _EngineBudget(expired=True)
    monkeypatch.setitem(sys.modules, "budget", engine)
    assert budget.shared() is engine and budget.expired() and budget.remaining() < 0
    res, timed = _search_with_stubs(monkeypatch)
    assert timed == [tune.candidates(8, 6144, 2560, 0)[0]]
    assert res.config == timed[0] and res.plan_us is not None and len(res.trials) == 1
    # start() goes to the engine's clock, not a private one
    budget.start(7.0)
    assert engine.started == [7.0]


def test_open_engine_budget_lets_every_candidate_run(monkeypatch):
    import sys

    from kernels import budget, tune

    budget.use(None)
    monkeypatch.setitem(sys.modules, "budget", _EngineBudget(expired=False))
    res, timed = _search_with_stubs(monkeypatch)
    assert timed == tune.candidates(8, 6144, 2560, 0) and len(timed) > 10


def test_explicit_budget_binding_wins(monkeypatch):
    import sys

    from kernels import budget

    monkeypatch.setitem(sys.modules, "budget", _EngineBudget(expired=False))
    mine = _EngineBudget(expired=True)
    budget.use(mine)
    try:
        assert budget.shared() is mine and budget.expired()
        _, timed = _search_with_stubs(monkeypatch)
        assert len(timed) == 1
    finally:
        budget.use(None)


def test_private_deadline_without_an_engine(monkeypatch):
    import sys

    from kernels import budget

    budget.use(None)
    monkeypatch.delitem(sys.modules, "budget", raising=False)
    assert budget.shared() is None
    budget.start(-1.0)
    try:
        assert budget.expired()
        _, timed = _search_with_stubs(monkeypatch)
        assert len(timed) == 1
    finally:
        budget.clear()
    assert not budget.expired()


def test_cli_line_for_cached_and_untimed_results():
    """A cache hit has no plan time (plan_us None); the CLI prints it
    instead of failing on a None format."""
    from kernels.tune import Result, _us_text

    cfg = {"kernel": 2}
    assert "cached" in _us_text(Result(cfg, float("nan"), None, cached=True))
    assert "-" in _us_text(Result(cfg, 5.0, None))
    assert "5.00" in _us_text(Result(cfg, 5.0, 6.0)) and "6.00" in _us_text(Result(cfg, 5.0, 6.0))


def test_search_cache_hit_is_not_timed(monkeypatch):
    from kernels import _lib, budget, tune

    class Props:
        gcnArchName = "gfx950"

    monkeypatch.setattr(tune.torch.cuda, "get_device_properties", lambda dev: Props())
    budget.use(None)
    cache = tune.TuneCache()
    calls = []
    build = lambda cfg: (lambda w: cfg)
    timer = lambda fn, rot: calls.append(fn(None)) or 2.0
    first = tune.search("matmul", 4, 2560, 4096, 0, "cuda:0", build, lambda fn: (True, ""), timer, [None],
                        cache=cache, limit=3)
    n = len(calls)
    again = tune.search("matmul", 4, 2560, 4096, 0, "cuda:0", build, lambda fn: (True, ""), timer, [None],
                        cache=cache, limit=3)
    assert len(calls) == n == 3 and again.cached and again.plan_us is None and again.config == first.config


def test_acceptance_rule_is_elementwise():
    """close_ok: |out - ref| <= 2e-2 + 1e-2|ref| at every element, NaN and
    infinities where the reference has them, plus the reference's global
    rule.  A wrong small-magnitude channel passes the global rule alone and
    must fail here."""
    import torch

    from kernels.tune import close_ok

    ref = torch.linspace(-4, 4, 64).reshape(2, 32).to(torch.bfloat16)
    assert close_ok(ref.clone(), ref)[0]
    bad = ref.clone()
    bad[0, 15] = ref[0, 15] + 0.05            # within 0.02 * max|ref| + 1e-3 = 0.081
    ok_global = (bad.float() - ref.float()).abs().max() <= 0.02 * ref.float().abs().max() + 1e-3
    assert ok_global and not close_ok(bad, ref)[0]
    nan_ref = ref.clone()
    nan_ref[1, 3] = float("nan")
    assert not close_ok(ref, nan_ref)[0]
    out = ref.clone()
    out[1, 3] = float("nan")
    assert close_ok(out, nan_ref)[0]
    inf_ref = ref.clone()
    inf_ref[0, 0] = float("inf")
    out = ref.clone()
    out[0, 0] = float("-inf")
    assert not close_ok(out, inf_ref)[0]
    out[0, 0] = float("inf")
    assert close_ok(out, inf_ref)[0]


def test_silu_mul_acceptance_allows_the_epilogue_rounding_chain():
    """close_ok(silu=True) also accepts elements within the reference's own
    gate/up rule 0.02|ref| + 1e-3.  The case measured on an MI355X: the
    exact gate sum 2.0078133 sits 8e-7 above the bf16 midpoint of 2 and
    2.015625; the kernel rounds it up, torch's fp32 sum rounds it down, and
    SiLU·mul with up = 3.765625 gives 6.71875 against 6.625, outside
    2e-2 + 1e-2|ref| (0.086) but within 0.02|ref| + 1e-3 (0.1335).  A plain
    projection keeps the tighter bar, and an error beyond both still fails."""
    import math

    import torch
    from kernels.tune import close_ok

    def swiglu(g, u):
        gb = float(torch.tensor(g).to(torch.bfloat16))
        s = float(torch.tensor(gb / (1.0 + math.exp(-gb))).to(torch.bfloat16))
        return float(torch.tensor(s * float(torch.tensor(u).to(torch.bfloat16))).to(torch.bfloat16))

    kernel_v = swiglu(2.015625, 3.765625)   # the gate rounded up (the exact sum's side)
    torch_v = swiglu(2.0, 3.765625)          # the gate rounded down
    assert (kernel_v, torch_v) == (6.71875, 6.625)
    ref = torch.full((4, 8), 1.0, dtype=torch.bfloat16)
    ref[2, 5] = torch_v
    out = ref.clone()
    out[2, 5] = kernel_v
    assert not close_ok(out, ref)[0]
    assert close_ok(out, ref, silu=True)[0]
    out[2, 5] = torch_v + 0.1875              # bf16 6.8125: beyond 0.02|ref| + 1e-3 as well
    assert not close_ok(out, ref, silu=True)[0]
    small = ref.clone()
    small[0, 0] = 0.0
    out = small.clone()
    out[0, 0] = 0.015                         # small |ref|: the 2e-2 absolute part still applies
    assert close_ok(out, small, silu=True)[0]
    out[0, 0] = 0.03
    assert not close_ok(out, small, silu=True)[0]


def test_pointwise_rule_of_the_m64_gateup_picker():
    """pointwise_ok: |out - ref| <= 0.02|ref| + 1e-3 at every element and
    everything finite (the reference's M = 64 gate/up acceptance).  An error
    the elementwise bar accepts near a small reference value fails it."""
    import torch
    from kernels.tune import close_ok, pointwise_ok

    ref = torch.linspace(-3, 3, 401)
    assert pointwise_ok(ref.clone(), ref)[0]
    out = ref.clone()
    out[200] += 5e-3                      # ref[200] = 0: allowed 1e-3 here, 2e-2 by close_ok
    assert close_ok(out, ref)[0] and not pointwise_ok(out, ref)[0]
    out = ref * (1 + 0.019)               # within 2% everywhere
    assert pointwise_ok(out, ref)[0]
    bad = ref.clone()
    bad[5] = float("inf")
    assert not pointwise_ok(bad, ref)[0]
    assert not pointwise_ok(ref[:10], ref)[0]


def test_validation_plan_of_the_tuner():
    """Candidates run on the call's weight and a second rotation weight; a
    gate/up projection of 64 rows or more runs on every distinct weight of
    the rotation under the pointwise rule as well."""
    from kernels.gemm import EPILOGUE_NONE, EPILOGUE_SILU_MUL, _validation_plan

    w, rot = object(), [object() for _ in range(5)]
    checks, strict = _validation_plan(32, EPILOGUE_SILU_MUL, w, [w] + rot)
    assert checks == [w, rot[0]] and not strict
    checks, strict = _validation_plan(64, EPILOGUE_NONE, rot[2], rot)
    assert checks == [rot[2], rot[1]] and not strict
    checks, strict = _validation_plan(64, EPILOGUE_SILU_MUL, w, [w] + rot + [rot[0]])
    assert checks == [w] + rot and strict
    checks, strict = _validation_plan(64, EPILOGUE_SILU_MUL, w, [w])
    assert checks == [w] and strict


def _margin_search(times_of, order_bias=None):
    """tune.search over the real candidate list of qkv at M = 8 with stub
    build / acceptance and a timer that returns ``times_of(index)`` for the
    candidate at that index of the list (the plan is index 0); with
    ``order_bias(index, call)`` the timer also sees how many timings came
    before, so a test can make a result depend on the order."""
    from kernels import budget, tune

    budget.use(None)
    budget.clear()
    cands = tune.candidates(8, 6144, 2560, 0)
    index = {id(c): i for i, c in enumerate(cands)}
    calls = []

    def build(cfg):
        i = next(j for j, c in enumerate(cands) if c == cfg)
        return lambda w: i

    def timer(fn, rot):
        i = fn(None)
        calls.append(i)
        t = times_of(i)
        return t * (order_bias(i, len(calls)) if order_bias else 1.0)

    res = tune.search("matmul", 8, 6144, 2560, 0, "cpu", build, lambda fn: (True, ""), timer, [None], cache=None)
    return res, cands, calls


def test_challenger_two_percent_faster_keeps_the_plan():
    """A candidate 2% faster than the plan in both orders does not clear the
    reference's 3% margin (m64_gateup_selection.py:124-128)."""
    res, cands, _ = _margin_search(lambda i: 1.0 if i == 0 else (0.98 if i == 3 else 1.2))
    assert res.config == cands[0] and res.us == res.plan_us == 1000.0
    assert [c[0] for c in res.confirmations] == [cands[3]]
    assert all(abs(r - 0.98) < 1e-9 for r in res.confirmations[0][1:])


def test_challenger_five_percent_faster_replaces_the_plan():
    res, cands, calls = _margin_search(lambda i: 1.0 if i == 0 else (0.95 if i == 5 else 1.2))
    assert res.config == cands[5] and abs(res.us - 950.0) < 1e-6 and res.plan_us == 1000.0
    # the sweep, then plan/challenger and challenger/plan
    assert calls[-4:] == [0, 5, 5, 0]


def test_challenger_must_clear_the_margin_in_both_orders():
    """5% faster when timed after the plan, 1.2% when timed first: kept out."""

    def times(i):
        return 1.0 if i == 0 else (0.95 if i == 4 else 1.2)

    res, cands, calls = _margin_search(times, order_bias=lambda i, n: 1.0)
    assert res.config == cands[4]
    # the sweep takes one timing per candidate; the challenger-first timing
    # of candidate 4 is then call len(cands) + 3
    n_sweep = len(calls)
    res, cands, calls = _margin_search(times, order_bias=lambda i, n: 1.04 if (i == 4 and n == n_sweep - 1) else 1.0)
    r1, r2 = res.confirmations[0][1:]
    assert r1 < 0.97 <= r2 and res.config == cands[0]


def test_best_of_several_challengers_by_worst_ratio():
    res, cands, _ = _margin_search(lambda i: {0: 1.0, 2: 0.96, 6: 0.90, 7: 0.93}.get(i, 1.3))
    assert res.config == cands[6]
    assert [c[0] for c in res.confirmations] == [cands[6], cands[7], cands[2]]


def test_downstream_check_of_gateup_candidates():
    """At 64 rows a gate/up candidate is also judged through the down
    projection that consumes it (m64_gateup_n32_selection.py:73-105): the
    down weights pair with the rotation's gate/up weights by position."""
    import torch

    from kernels.gemm import _down_for, downstream_ok

    g = torch.Generator().manual_seed(5)
    ref = torch.randn((64, 96), generator=g).to(torch.bfloat16)
    wd = (torch.randn((40, 96), generator=g) * 0.05).to(torch.bfloat16)
    assert downstream_ok(ref.clone(), ref, wd)[0]
    bad = ref.clone()
    bad[7] = bad[7] * 1.3                      # one whole row 30% off: the down rows move with it
    ok, why = downstream_ok(bad, ref, wd)
    assert not ok and why.startswith("down projection")
    w, rot = object(), [object() for _ in range(3)]
    downs = ["d0", "d1", "d2"]
    assert _down_for([rot[1], rot[2]], rot[1], rot, downs) == ["d1", "d2"]
    assert _down_for([w, rot[0]], w, rot, downs) == ["d0", "d0"]
    assert _down_for([w], w, rot, None) == []
    t = torch.zeros(1)
    assert _down_for([w, rot[0]], w, rot, t) == [t, t]
    import pytest

    with pytest.raises(ValueError):
        _down_for([w], w, rot, ["d0"])
