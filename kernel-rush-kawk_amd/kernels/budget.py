"""Warm-up time budget of the tuning pickers: one clock with the engine's.

The reference engine starts a single deadline, ``budget.start(PICKER_BUDGET_S)``
(engine/engine.py:44, 504), in its own module ``budget`` (engine/budget.py),
and every picker polls that module (engine/kernels/gemm.py:437, 478, 541).
This module is what this library's pickers poll (kernels/tune.py), and it
reads the engine's clock whenever there is one:

* :func:`use` binds a budget object explicitly (any object with
  ``start(seconds)``, ``expired()`` and ``remaining()``);
* otherwise, when a module named ``budget`` with those functions is loaded
  (the engine's, imported as ``budget`` from the engine directory), it is the
  clock — so ``budget.start(120)`` in the engine bounds this library's
  tuning with no further wiring;
* otherwise (stand-alone use: the tuner's command line, bench.py) a private
  deadline is kept here.

:func:`start` and :func:`clear` act on whichever clock is in use.  With no
deadline set, every candidate is tried.
"""

from __future__ import annotations

import sys
import time

_deadline: float | None = None
_bound = None
_API = ("start", "expired", "remaining")


def _has_api(obj) -> bool:
    return all(callable(getattr(obj, name, None)) for name in _API)


def use(clock) -> None:
    """Poll ``clock`` from now on (``None`` unbinds: back to discovery)."""
    global _bound
    if clock is not None and not _has_api(clock):
        raise ValueError(f"a budget needs callables {', '.join(_API)}")
    _bound = clock


def shared():
    """The external clock in use, or None when the private deadline is."""
    if _bound is not None:
        return _bound
    mod = sys.modules.get("budget")
    if mod is None or mod is sys.modules.get(__name__) or not _has_api(mod):
        return None
    return mod


def start(seconds: float) -> None:
    global _deadline
    clock = shared()
    if clock is not None:
        clock.start(seconds)
    else:
        _deadline = time.monotonic() + seconds


def clear() -> None:
    """No deadline.  An external clock without a ``clear`` is given an
    unbounded one."""
    global _deadline
    clock = shared()
    if clock is None:
        _deadline = None
    elif callable(getattr(clock, "clear", None)):
        clock.clear()
    else:
        clock.start(float("inf"))


def expired() -> bool:
    clock = shared()
    if clock is not None:
        return bool(clock.expired())
    return _deadline is not None and time.monotonic() > _deadline


def remaining() -> float:
    clock = shared()
    if clock is not None:
        return float(clock.remaining())
    return float("inf") if _deadline is None else _deadline - time.monotonic()
