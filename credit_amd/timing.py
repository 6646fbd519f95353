"""Event-timed trials of library calls on the MI355X.

Two effects decide what a timing loop over these kernels measures:

* the HBM clock ramp: after an idle period the first 10-20 ms of HBM-bound
  work run up to 35% slow (C2 LayerNorm forward, per 100-call block from a
  cold start: 64.9, 48.1, then 47.3-47.6 us per call), so every timed block
  follows a settle phase of back-to-back calls;
* host-bound launches: a Python launcher with tensor checks takes about as
  long as a 47 us kernel, so the calls timed here are ``hip_lib.bind``
  closures (one ctypes call each) issued back to back.

A measurement is ``trials`` blocks of ``iters`` calls, each block bracketed
by HIP events on the current torch stream (the stream the library launches
on); the per-call time of a block is one sample.  The summary is the median
sample and the 20th / 80th percentiles (``statistics.quantiles`` over the
samples, inclusive method: the smallest sample is the 0th percentile, the
largest the 100th, linear in between).  The reference's harness times one event-bracketed loop per
variant (src/workloads/layernorm_backward.cu:150-175) and summarises repeated
runs by median and quantiles (dsmem_eval/runner.py:130-182); this module is
this build's form of both.
"""
from __future__ import annotations

import math
import statistics
import time
from dataclasses import dataclass
from typing import Callable

import torch

Call = Callable[[int], object]


@dataclass(frozen=True)
class TrialStats:
    """Per-call milliseconds of `trials` blocks of `iters` calls each."""

    samples_ms: tuple[float, ...]
    iters: int

    @property
    def trials(self) -> int:
        return len(self.samples_ms)

    def _cuts(self) -> tuple[float, float]:
        finite = sorted(v for v in self.samples_ms if math.isfinite(v))
        if not finite:
            return math.nan, math.nan
        if len(finite) == 1:
            return finite[0], finite[0]
        q = statistics.quantiles(finite, n=5, method="inclusive")  # 20/40/60/80 %
        return q[0], q[3]

    @property
    def median_ms(self) -> float:
        finite = [v for v in self.samples_ms if math.isfinite(v)]
        return statistics.median(finite) if finite else math.nan

    @property
    def p20_ms(self) -> float:
        return self._cuts()[0]

    @property
    def p80_ms(self) -> float:
        return self._cuts()[1]

    def as_dict(self, digits: int = 6) -> dict:
        return {"median_ms": round(self.median_ms, digits), "p20_ms": round(self.p20_ms, digits),
                "p80_ms": round(self.p80_ms, digits), "trials": self.trials, "iters": self.iters}


def settle(call: Call, settle_ms: float, start: int = 0, batch: int = 8) -> int:
    """Issue calls back to back for settle_ms of wall time, synchronising
    every `batch` calls so that wall time is GPU time.  Returns the next
    call index."""
    i = start
    deadline = time.perf_counter() + settle_ms / 1e3
    while time.perf_counter() < deadline:
        for _ in range(batch):
            call(i)
            i += 1
        torch.cuda.synchronize()
    return i


def timed_block(call: Call, iters: int, start: int = 0) -> tuple[float, float]:
    """(wall ms, event ms) per call of `iters` back-to-back calls, the
    device synchronised on both sides."""
    torch.cuda.synchronize()
    begin = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    begin.record()
    for k in range(iters):
        call(start + k)
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return wall / iters, begin.elapsed_time(end) / iters


def run_trials(call: Call, trials: int, iters: int, warmup: int = 0, settle_ms: float = 0.0,
               start: int = 0) -> TrialStats:
    """Settle, warm up, then time `trials` blocks of `iters` calls.  The
    call index keeps counting across phases, so a caller rotating buffer
    sets by index never repeats a set back to back."""
    if trials < 1 or iters < 1:
        raise ValueError("trials and iters must be >= 1")
    i = settle(call, settle_ms, start) if settle_ms > 0 else start
    for _ in range(warmup):
        call(i)
        i += 1
    samples = []
    for _ in range(trials):
        _, ms = timed_block(call, iters, i)
        samples.append(ms)
        i += iters
    return TrialStats(tuple(samples), iters)
