"""Timing protocol (`kernelforge/bench.py:113-161`, organizer `:463-583`).

Event-timed calls on the current stream, warm-up first, interleaved round-robin over
candidates with the visiting order rotated each round, medians reported. (The NVML
power sampling and clock locking of the reference are NVIDIA-only and not carried.)
"""
from __future__ import annotations

import dataclasses
import statistics
from typing import Callable, Dict, List

import torch


@dataclasses.dataclass
class Timing:
    samples_ms: List[float]

    @property
    def median_ms(self) -> float:
        return statistics.median(self.samples_ms)

    @property
    def mean_ms(self) -> float:
        return statistics.fmean(self.samples_ms)

    @property
    def min_ms(self) -> float:
        return min(self.samples_ms)

    @property
    def p90_ms(self) -> float:
        s = sorted(self.samples_ms)
        return s[min(len(s) - 1, int(0.9 * (len(s) - 1)))]

    @property
    def spread(self) -> float:
        return self.p90_ms / self.min_ms if self.min_ms else float("nan")


def time_block(fn: Callable[[], object], iters: int) -> List[float]:
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    torch.cuda.synchronize()
    for i in range(iters):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def compare(candidates: Dict[str, Callable[[], object]], warmup: int = 20,
            repeats: int = 50, rounds: int = 3) -> Dict[str, Timing]:
    names = list(candidates)
    with torch.inference_mode():
        for name in names:
            for _ in range(warmup):
                candidates[name]()
        torch.cuda.synchronize()
        samples: Dict[str, List[float]] = {n: [] for n in names}
        for r in range(rounds):
            order = names[r % len(names):] + names[:r % len(names)]
            for name in order:
                samples[name].extend(time_block(candidates[name], repeats))
    return {n: Timing(samples[n]) for n in names}
