"""Kernel timing with HIP events.

Launches are asynchronous, so wall-clock around a call measures enqueueing.
As in the reference (kernelforge/benchmark/runner.py:123-191), each timed
iteration is bracketed by events recorded on the current stream, the stream
is synchronised once after the loop, and the samples are summarised as a
distribution (median ranked, never the minimum).

Two MI355X-specific changes to the cache flush before every iteration:

* It covers the whole L2 *and* the 256 MiB Infinity Cache (MALL). Every
  working set in the BASELINE configurations except the 11008-wide softmax
  fits in the MALL, so an L2-sized flush (the reference's) would report
  cache bandwidth as HBM bandwidth.
* It *reads* the flush buffer instead of zeroing it. Zeroing leaves hundreds
  of MiB of dirty lines in the memory-side cache, and their write-back then
  competes with the measured kernel for HBM.

The flush is enqueued before the start event on the same in-order stream,
so it is not part of the measured interval -- and because it keeps the GPU
busy while the host enqueues the next call, host-side wrapper overhead is
not measured either.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np
import torch

from kernelforge.runtime.env import device_caps

DEFAULT_WARMUP = 25
DEFAULT_ITERATIONS = 200

#: hipEvent elapsed-time resolution is about a microsecond; medians at or
#: below this are reported but not compared.
TIMER_RESOLUTION_MS = 0.002


@dataclass(frozen=True)
class TimingResult:
    """Summary of one timing run. All times are milliseconds."""

    median_ms: float
    mean_ms: float
    std_ms: float
    min_ms: float
    max_ms: float
    p95_ms: float
    p99_ms: float
    warmup: int
    iterations: int
    timer: str
    flushed_l2: bool
    samples_ms: tuple[float, ...] = field(default=(), repr=False)

    @property
    def at_timer_resolution(self) -> bool:
        return self.timer == "hip_event" and self.median_ms <= TIMER_RESOLUTION_MS

    @property
    def median_us(self) -> float:
        return self.median_ms * 1e3

    def as_dict(self) -> dict[str, float | int | str | bool]:
        return {
            "median_ms": self.median_ms,
            "mean_ms": self.mean_ms,
            "std_ms": self.std_ms,
            "min_ms": self.min_ms,
            "max_ms": self.max_ms,
            "p95_ms": self.p95_ms,
            "p99_ms": self.p99_ms,
            "warmup": self.warmup,
            "iterations": self.iterations,
            "timer": self.timer,
            "flushed_l2": self.flushed_l2,
        }


def summarize(
    samples_ms: list[float] | np.ndarray,
    *,
    warmup: int,
    iterations: int,
    timer: str,
    flushed_l2: bool,
    keep_samples: bool = False,
) -> TimingResult:
    """Summarise per-iteration timings (numpy linear-interpolation percentiles)."""
    arr = np.asarray(samples_ms, dtype=np.float64)
    if arr.size == 0:
        raise ValueError("cannot summarize an empty set of timing samples")
    p95, p99 = (float(x) for x in np.percentile(arr, [95, 99]))
    return TimingResult(
        median_ms=float(np.median(arr)),
        mean_ms=float(arr.mean()),
        std_ms=float(arr.std(ddof=1)) if arr.size > 1 else 0.0,
        min_ms=float(arr.min()),
        max_ms=float(arr.max()),
        p95_ms=p95,
        p99_ms=p99,
        warmup=warmup,
        iterations=iterations,
        timer=timer,
        flushed_l2=flushed_l2,
        samples_ms=tuple(float(x) for x in arr) if keep_samples else (),
    )


class CacheFlush:
    """Evicts every L2 and the Infinity Cache by reading a buffer that covers them.

    ``flush()`` enqueues one reduction over the buffer on the current stream;
    the result lands in a preallocated scalar, so nothing is allocated per call.
    """

    def __init__(self, device: torch.device) -> None:
        nbytes = device_caps(device).flush_bytes
        self.buffer = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
        self._sink = torch.empty((), dtype=torch.float32, device=device)

    def flush(self) -> None:
        torch.sum(self.buffer, dim=0, out=self._sink)

    # The reference zeroes its flush buffer with ``cache.zero_()``; keep that
    # spelling working for callers written against it.
    zero_ = flush


_FLUSH: dict[int, CacheFlush] = {}


def flush_buffer(device: torch.device) -> CacheFlush:
    """The per-device cache flush, created once."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    flusher = _FLUSH.get(index)
    if flusher is None:
        flusher = CacheFlush(torch.device("cuda", index))
        _FLUSH[index] = flusher
    return flusher


def benchmark(
    fn,
    *,
    warmup: int = DEFAULT_WARMUP,
    iterations: int = DEFAULT_ITERATIONS,
    device: torch.device | str | None = None,
    flush_l2: bool = True,
    keep_samples: bool = False,
) -> TimingResult:
    """Time ``fn`` (no arguments) and return the latency distribution.

    Without a GPU in play this falls back to ``time.perf_counter`` and labels
    the result ``perf_counter``, so a CPU time can never pass for a GPU one
    (runner.py:153-166).
    """
    if warmup < 0:
        raise ValueError(f"warmup must be non-negative, got {warmup}")
    if iterations < 1:
        raise ValueError(f"iterations must be at least 1, got {iterations}")

    resolved = torch.device(device) if device is not None else None
    use_gpu = torch.cuda.is_available() and (resolved is None or resolved.type == "cuda")

    for _ in range(warmup):
        fn()

    if not use_gpu:
        samples = []
        for _ in range(iterations):
            t0 = time.perf_counter()
            fn()
            samples.append((time.perf_counter() - t0) * 1e3)
        return summarize(
            samples,
            warmup=warmup,
            iterations=iterations,
            timer="perf_counter",
            flushed_l2=False,
            keep_samples=keep_samples,
        )

    gpu = resolved if resolved is not None else torch.device("cuda", torch.cuda.current_device())
    torch.cuda.synchronize(gpu)
    cache = flush_buffer(gpu) if flush_l2 else None
    start = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
    for i in range(iterations):
        if cache is not None:
            cache.flush()
        start[i].record()
        fn()
        end[i].record()
    torch.cuda.synchronize(gpu)
    samples = [start[i].elapsed_time(end[i]) for i in range(iterations)]
    return summarize(
        samples,
        warmup=warmup,
        iterations=iterations,
        timer="hip_event",
        flushed_l2=flush_l2,
        keep_samples=keep_samples,
    )


def cross_check_median_ms(fn, *, warmup: int = DEFAULT_WARMUP, min_run_time: float = 1.0) -> float:
    """Independent median latency from ``torch.utils.benchmark`` (runner.py:194-207)."""
    import torch.utils.benchmark as torch_benchmark

    for _ in range(warmup):
        fn()
    timer = torch_benchmark.Timer(stmt="fn()", globals={"fn": fn})
    return float(timer.blocked_autorange(min_run_time=min_run_time).median) * 1e3
