"""Warm-up time budget shared by the tuning pickers (reference
engine/budget.py:1-27).

The engine calls ``start(seconds)`` before the first pick; each picker keeps
trying candidate configurations while ``expired()`` is false and otherwise
keeps the best one measured so far (the dispatch table's configuration is
always measured first).  With no deadline set, every candidate is tried.
"""

from __future__ import annotations

import time

_deadline: float | None = None


def start(seconds: float) -> None:
    global _deadline
    _deadline = time.monotonic() + seconds


def clear() -> None:
    global _deadline
    _deadline = None


def expired() -> bool:
    return _deadline is not None and time.monotonic() > _deadline


def remaining() -> float:
    return float("inf") if _deadline is None else _deadline - time.monotonic()
