"""Device-side timing shared by ``bench.py`` and the benchmark harness.

A :class:`PhaseClock` records a HIP event on the current stream at every
named mark; once the last mark has completed, each phase's time is the
elapsed time between its mark and the one before. Recording events costs a
few microseconds of host time per mark and nothing on the device, so a step
can be split into phases (forward, backward) without synchronising inside it.
"""

from __future__ import annotations

import contextlib
import gc
import statistics
from typing import Callable, Iterator

import torch


@contextlib.contextmanager
def paused_collector() -> Iterator[None]:
    """Run a full garbage collection, then keep the collector off until the
    block ends. With torch loaded the interpreter tracks about 170k objects,
    and a generation-2 collection of them takes about 40 ms of host time; one
    that lands inside a timed step stalls the launches behind it and
    inflates that step's time by the same amount. The timed blocks create
    no reference cycles worth collecting, so pausing the collector there
    leaks nothing."""
    enabled = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        if enabled:
            gc.enable()


@contextlib.contextmanager
def collected_collector() -> Iterator[None]:
    """Run a full garbage collection and leave the collector as it was, so
    that the block starts from an empty young generation but still pays any
    collection its own allocations trigger, as a training loop does."""
    gc.collect()
    yield


class PhaseClock:
    """Named marks on the current stream of the current device."""

    def __init__(self) -> None:
        self._marks: list[tuple[str, torch.cuda.Event]] = []

    def mark(self, name: str) -> None:
        event = torch.cuda.Event(enable_timing=True)
        event.record()
        self._marks.append((name, event))

    def phases(self) -> dict[str, float]:
        """Milliseconds of every phase, keyed by the mark that ends it
        (waits for the last mark)."""
        if not self._marks:
            return {}
        self._marks[-1][1].synchronize()
        return {name: before.elapsed_time(event)
                for (_, before), (name, event) in zip(self._marks, self._marks[1:])}


def time_phases(step: Callable[[PhaseClock], None], warmup: int, iterations: int,
                before: Callable[[], None] | None = None) -> dict[str, list[float]]:
    """Run ``step`` ``warmup`` times untimed, then ``iterations`` times with a
    fresh clock each; ``step`` marks "start" first and then the end of each
    of its phases. ``before`` (e.g. clearing gradients) runs ahead of every
    step, outside the marks. The collector is paused over the measured
    iterations (:func:`paused_collector`). Returns each phase's milliseconds
    per iteration."""
    for _ in range(warmup):
        if before is not None:
            before()
        step(PhaseClock())
    torch.cuda.synchronize()
    samples: dict[str, list[float]] = {}
    with paused_collector():
        for _ in range(iterations):
            if before is not None:
                before()
            clock = PhaseClock()
            step(clock)
            for name, ms in clock.phases().items():
                samples.setdefault(name, []).append(ms)
    return samples


def mean(values: list[float]) -> float:
    return statistics.fmean(values) if values else 0.0
