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
