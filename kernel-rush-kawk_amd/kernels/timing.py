"""Graph-replay timing shared by the tuner, the pickers and bench.py.

A call sequence is recorded once in a HIP graph and the graph is replayed;
the time per call is the median replay time divided by the number of calls.
Replaying removes the host's launch cost from the measurement, and a
sequence that cycles through distinct weight tensors (every layer's copy of
a projection) keeps the weights out of the caches, so the figure is the one
a decode step sees.  This is the measurement method of the reference's
picker timer (engine/kernels/gemm.py:378-414); the code here is this
library's own.
"""

from __future__ import annotations

import itertools
import math
import statistics
from typing import Callable, Sequence

import torch


class GraphReplay:
    """``calls`` (zero-argument callables) recorded in one graph.

    The first ``warmup`` calls of the cycled sequence run eagerly on a side
    stream before capture, so lazily created state (workspaces, library
    handles) exists before recording starts.
    """

    def __init__(self, calls: Sequence[Callable[[], object]], warmup: int = 3):
        if not calls:
            raise ValueError("need at least one call to time")
        self.calls = list(calls)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for call in itertools.islice(itertools.cycle(self.calls), warmup):
                call()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for call in self.calls:
                call()
        self.replay()
        torch.cuda.synchronize()

    def replay(self) -> None:
        self.graph.replay()

    def ms_per_call(self, reps: int = 5, warm_ms: float = 10.0) -> float:
        """Median over ``reps`` timed replays, divided by the number of calls.
        Untimed replays covering about ``warm_ms`` of GPU time run first: a
        GPU that idled while the graph was built runs its first milliseconds
        slower (measured on an MI355X: with one untimed replay, the first of
        several timings of a graph came out up to 8% above the rest, with
        2 ms of replays up to 3%, with 10 ms within 0.5%).  The timed replays
        are enqueued back to back and read after one synchronisation."""
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        self.replay()
        end.record()
        torch.cuda.synchronize()
        one = max(begin.elapsed_time(end), 1e-3)
        for _ in range(min(64, math.ceil(warm_ms / one))):
            self.replay()
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for begin, end in marks:
            begin.record()
            self.replay()
            end.record()
        torch.cuda.synchronize()
        return statistics.median(begin.elapsed_time(end) for begin, end in marks) / len(self.calls)


def replay_ms(calls: Sequence[Callable[[], object]], reps: int = 5) -> float:
    """Milliseconds per call of ``calls`` replayed from one graph."""
    return GraphReplay(calls).ms_per_call(reps)


def rotation_calls(fn: Callable, count: int, rotate: Sequence | None = None) -> list:
    """``count`` calls of ``fn``: ``fn(w)`` over the weights of ``rotate`` in
    turn, or ``fn()`` when there is no rotation."""
    if not rotate:
        return [fn] * count
    return [(lambda w=w: fn(w)) for w in itertools.islice(itertools.cycle(rotate), count)]
