"""Kernel timing on MI355X: HIP events on the launching stream, caches flushed.

A launch returns before the kernel runs, so a host clock around a call times
the enqueue. Each timed iteration here is therefore bracketed by two HIP
events recorded on the stream the kernel is launched on (torch's current
stream), and the stream is synchronised once, after the loop. The samples are
summarised as a distribution; ranking uses the median
(kernelforge/benchmark/runner.py:123-191 defines the same protocol).

What is specific to this GPU:

* **The flush covers L2 and the Infinity Cache.** An MI355X has 8 XCDs with
  a 4 MiB L2 each and a 256 MiB memory-side Infinity Cache (MALL). Every
  BASELINE working set but one fits in the MALL, so flushing only L2 would
  report MALL bandwidth as HBM bandwidth. :class:`CacheFlush` streams a
  buffer of L2 + MALL bytes through a reduction before every iteration.
  Reading (not zeroing) leaves no dirty lines whose write-back would compete
  with the measured kernel.
* **Events are pooled.** One ring of timing-enabled events per (device,
  size) is created once and reused, so a tuning sweep of hundreds of
  candidates does not create and destroy hundreds of thousands of events.
* **Dispatch overlap.** The flush keeps the GPU busy while the host enqueues
  the start event and the kernel, so host-side wrapper time stays outside
  the measured interval as long as it is shorter than the flush.

Without a GPU the harness times with ``time.perf_counter`` and labels the
result ``perf_counter``, so a CPU time can never pass for a GPU one.
"""

from __future__ import annotations

import time
from collections.abc import Callable
from dataclasses import dataclass, field

import numpy as np
import torch

from kernelforge.runtime.env import device_caps

DEFAULT_WARMUP = 25
DEFAULT_ITERATIONS = 200

#: HIP event timestamps resolve to about a microsecond; medians at or below
#: this are reported but must not be compared between implementations.
TIMER_RESOLUTION_MS = 0.002

TIMER_HIP_EVENT = "hip_event"
TIMER_PERF_COUNTER = "perf_counter"


@dataclass(frozen=True)
class TimingResult:
    """A latency distribution. All times are milliseconds."""

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
        """True when the median is too short for event timestamps to rank it."""
        return self.timer in (TIMER_HIP_EVENT, "cuda_event") and self.median_ms <= TIMER_RESOLUTION_MS

    @property
    def median_us(self) -> float:
        return 1e3 * self.median_ms

    def as_dict(self) -> dict[str, float | int | str | bool]:
        keys = ("median_ms", "mean_ms", "std_ms", "min_ms", "max_ms", "p95_ms", "p99_ms",
                "warmup", "iterations", "timer", "flushed_l2")
        return {k: getattr(self, k) for k in keys}


def summarize(
    samples_ms: list[float] | np.ndarray,
    *,
    warmup: int,
    iterations: int,
    timer: str,
    flushed_l2: bool,
    keep_samples: bool = False,
) -> TimingResult:
    """Distribution of per-iteration times.

    Quantiles interpolate linearly between order statistics (numpy's
    default); the standard deviation is the sample one (n - 1).
    """
    data = np.sort(np.asarray(samples_ms, dtype=np.float64).ravel())
    if data.size == 0:
        raise ValueError("cannot summarize an empty set of timing samples")
    median, p95, p99 = np.quantile(data, (0.5, 0.95, 0.99))
    return TimingResult(
        median_ms=float(median),
        mean_ms=float(data.mean()),
        std_ms=float(data.std(ddof=1)) if data.size > 1 else 0.0,
        min_ms=float(data[0]),
        max_ms=float(data[-1]),
        p95_ms=float(p95),
        p99_ms=float(p99),
        warmup=warmup,
        iterations=iterations,
        timer=timer,
        flushed_l2=flushed_l2,
        samples_ms=tuple(map(float, np.asarray(samples_ms, dtype=np.float64).ravel()))
        if keep_samples else (),
    )


class CacheFlush:
    """Evicts every XCD's L2 and the Infinity Cache by reading through them.

    ``flush()`` enqueues one reduction over an L2 + MALL sized buffer on the
    current stream, into a preallocated scalar: nothing is allocated per call.
    """

    def __init__(self, device: torch.device) -> None:
        self.nbytes = device_caps(device).flush_bytes
        self.buffer = torch.ones(self.nbytes // 4, dtype=torch.float32, device=device)
        self._sink = torch.empty((), dtype=torch.float32, device=device)

    def flush(self) -> None:
        torch.sum(self.buffer, dim=0, out=self._sink)

    #: The reference spells its flush ``cache.zero_()``; callers written
    #: against it keep working.
    zero_ = flush


_FLUSHES: dict[int, CacheFlush] = {}


def _index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def flush_buffer(device: torch.device) -> CacheFlush:
    """The per-device cache flush, created on first use."""
    idx = _index(device)
    if idx not in _FLUSHES:
        _FLUSHES[idx] = CacheFlush(torch.device("cuda", idx))
    return _FLUSHES[idx]


class _EventRing:
    """``size`` pairs of timing events on one device, reused across calls."""

    _rings: dict[tuple[int, int], _EventRing] = {}

    def __init__(self, size: int) -> None:
        self.start = [torch.cuda.Event(enable_timing=True) for _ in range(size)]
        self.end = [torch.cuda.Event(enable_timing=True) for _ in range(size)]

    @classmethod
    def get(cls, device: torch.device, size: int) -> _EventRing:
        key = (_index(device), size)
        if key not in cls._rings:
            with torch.cuda.device(key[0]):
                cls._rings[key] = cls(size)
        return cls._rings[key]

    def elapsed_ms(self) -> list[float]:
        return [s.elapsed_time(e) for s, e in zip(self.start, self.end)]


def _time_on_device(fn: Callable[[], object], device: torch.device, iterations: int,
                    flush: CacheFlush | None) -> list[float]:
    ring = _EventRing.get(device, iterations)
    stream = torch.cuda.current_stream(device)
    torch.cuda.synchronize(device)
    for start, end in zip(ring.start, ring.end):
        if flush is not None:
            flush.flush()
        start.record(stream)
        fn()
        end.record(stream)
    torch.cuda.synchronize(device)
    return ring.elapsed_ms()


def _time_on_host(fn: Callable[[], object], iterations: int) -> list[float]:
    samples = []
    clock = time.perf_counter
    for _ in range(iterations):
        begin = clock()
        fn()
        samples.append((clock() - begin) * 1e3)
    return samples


def benchmark(
    fn: Callable[[], object],
    *,
    warmup: int = DEFAULT_WARMUP,
    iterations: int = DEFAULT_ITERATIONS,
    device: torch.device | str | None = None,
    flush_l2: bool = True,
    keep_samples: bool = False,
) -> TimingResult:
    """Time ``fn`` (no arguments: bind inputs beforehand) ``iterations`` times.

    ``flush_l2`` flushes L2 and the Infinity Cache before every iteration on a
    GPU; on the CPU path nothing is flushed and the result says so.
    """
    if warmup < 0:
        raise ValueError(f"warmup must be non-negative, got {warmup}")
    if iterations < 1:
        raise ValueError(f"iterations must be at least 1, got {iterations}")
    target = torch.device(device) if device is not None else None
    on_gpu = torch.cuda.is_available() and (target is None or target.type == "cuda")
    for _ in range(warmup):
        fn()
    if on_gpu:
        gpu = target if target is not None else torch.device("cuda", torch.cuda.current_device())
        samples = _time_on_device(fn, gpu, iterations, flush_buffer(gpu) if flush_l2 else None)
        timer, flushed = TIMER_HIP_EVENT, flush_l2
    else:
        samples, timer, flushed = _time_on_host(fn, iterations), TIMER_PERF_COUNTER, False
    return summarize(samples, warmup=warmup, iterations=iterations, timer=timer,
                     flushed_l2=flushed, keep_samples=keep_samples)


def cross_check_median_ms(fn: Callable[[], object], *, warmup: int = DEFAULT_WARMUP,
                          min_run_time: float = 1.0) -> float:
    """A second opinion on the median (ms) from ``torch.utils.benchmark``.

    It synchronises and replicates on its own, unflushed; the GPU tests use it
    to check this harness, never to report numbers.
    """
    import torch.utils.benchmark as torch_benchmark

    for _ in range(warmup):
        fn()
    measured = torch_benchmark.Timer(stmt="fn()", globals={"fn": fn}).blocked_autorange(
        min_run_time=min_run_time)
    return 1e3 * float(measured.median)
