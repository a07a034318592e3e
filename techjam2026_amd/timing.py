"""GPU timing for comparing forwards: the protocol of `kernelforge/bench.py:113-161` and
the organizer's benchmark (`torch_transformer_benchmark.py:463-583`).

Protocol: every candidate is warmed up first; then the candidates are visited in rounds,
each round in a rotated order (round r starts at candidate r), and each visit times a
burst of calls with HIP events recorded on the current stream around every call. A
candidate's figure is the median over all its calls. Rotating the order spreads clock
and thermal drift over the candidates instead of charging it to whichever runs last.

The reference also samples NVML power and locks clocks; neither exists on this path.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Callable, Dict, List, Sequence

import torch


def _quantile(sorted_ms: Sequence[float], q: float) -> float:
    """Linear-interpolated quantile of ascending samples (q in [0, 1])."""
    if not sorted_ms:
        return float("nan")
    pos = q * (len(sorted_ms) - 1)
    lo = math.floor(pos)
    hi = min(lo + 1, len(sorted_ms) - 1)
    return sorted_ms[lo] + (sorted_ms[hi] - sorted_ms[lo]) * (pos - lo)


@dataclasses.dataclass(frozen=True)
class Timing:
    """Per-call durations (ms) of one candidate, with the visit (round) each came from."""

    samples_ms: List[float]
    rounds: List[int] = dataclasses.field(default_factory=list)

    @property
    def _sorted(self) -> List[float]:
        return sorted(self.samples_ms)

    @property
    def median_ms(self) -> float:
        return _quantile(self._sorted, 0.5)

    @property
    def min_ms(self) -> float:
        return min(self.samples_ms) if self.samples_ms else float("nan")

    @property
    def mean_ms(self) -> float:
        return sum(self.samples_ms) / len(self.samples_ms) if self.samples_ms else float("nan")

    @property
    def p90_ms(self) -> float:
        return _quantile(self._sorted, 0.9)

    @property
    def spread(self) -> float:
        """p90 over the fastest call: 1.0 for a perfectly steady candidate."""
        best = self.min_ms
        return self.p90_ms / best if best and best == best else float("nan")

    def round_medians(self) -> List[float]:
        """Median of each visit, in round order (a drift check)."""
        out = []
        for r in sorted(set(self.rounds)):
            out.append(_quantile(sorted(s for s, k in zip(self.samples_ms, self.rounds) if k == r), 0.5))
        return out


class EventClock:
    """A reusable pool of HIP event pairs; `measure(fn, n)` times n calls of fn, one
    event pair per call, on the current stream, and returns their durations in ms."""

    def __init__(self, capacity: int = 0):
        self._pairs: List[tuple] = []
        self._grow(capacity)

    def _grow(self, n: int) -> None:
        while len(self._pairs) < n:
            self._pairs.append((torch.cuda.Event(enable_timing=True),
                                torch.cuda.Event(enable_timing=True)))

    def measure(self, fn: Callable[[], object], n: int) -> List[float]:
        self._grow(n)
        torch.cuda.synchronize()
        for begin, end in self._pairs[:n]:
            begin.record()
            fn()
            end.record()
        torch.cuda.synchronize()
        return [begin.elapsed_time(end) for begin, end in self._pairs[:n]]


def visit_order(names: Sequence[str], rounds: int) -> List[List[str]]:
    """The candidates visited in each round: round r starts at candidate r (mod count)."""
    names = list(names)
    if not names:
        return [[] for _ in range(rounds)]
    return [names[r % len(names):] + names[:r % len(names)] for r in range(rounds)]


def compare(candidates: Dict[str, Callable[[], object]], warmup: int = 20,
            repeats: int = 50, rounds: int = 3) -> Dict[str, Timing]:
    """Warm every candidate up, then `rounds` rotated visits of `repeats` timed calls each."""
    names = list(candidates)
    clock = EventClock(repeats)
    samples: Dict[str, List[float]] = {n: [] for n in names}
    visit: Dict[str, List[int]] = {n: [] for n in names}
    with torch.inference_mode():
        for n in names:
            for _ in range(warmup):
                candidates[n]()
        torch.cuda.synchronize()
        for r, order in enumerate(visit_order(names, rounds)):
            for n in order:
                got = clock.measure(candidates[n], repeats)
                samples[n] += got
                visit[n] += [r] * len(got)
    return {n: Timing(samples[n], visit[n]) for n in names}
