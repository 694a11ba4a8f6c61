"""What ran: device kernels per call and their device time, from ``torch.profiler``.

The event harness says how long a call takes; this says which kernels the
call launched, which is the evidence for fusion (the unfused linear + bias +
GELU launches at least three kernels per call, the fused one exactly one;
kernelforge/profiling/pytorch_profiler.py:53-135 records the same). On ROCm
the profiler's device activity comes from the HIP runtime's own tracing, so
launches made through ``libkernelforge_hip.so`` are attributed the same way
as torch's.

The raw device events are grouped here by kernel name, not through the
profiler's own averaging tables, so a record is exactly (name, number of
device executions, summed device microseconds). Tracing perturbs timing: use
these figures for attribution, the event harness for latency.
"""

from __future__ import annotations

from collections import defaultdict
from collections.abc import Callable, Iterable
from dataclasses import dataclass
from pathlib import Path

import torch
from torch.autograd import DeviceType


@dataclass(frozen=True)
class KernelRecord:
    name: str
    launches: int
    device_time_us: float


@dataclass(frozen=True)
class ProfileResult:
    label: str
    iterations: int
    kernels: tuple[KernelRecord, ...]
    trace_path: Path | None = None

    def _per_call(self, total: float) -> float:
        return total / self.iterations if self.iterations else 0.0

    @property
    def launches_per_iteration(self) -> float:
        return self._per_call(sum(k.launches for k in self.kernels))

    @property
    def device_time_per_iteration_us(self) -> float:
        return self._per_call(sum(k.device_time_us for k in self.kernels))

    def render(self, limit: int = 10) -> str:
        out = [self.label,
               f"  kernel launches per call : {self.launches_per_iteration:.2f}",
               f"  device time per call     : {self.device_time_per_iteration_us:.1f} us"]
        shown = self.kernels[:limit]
        if shown:
            total = sum(k.device_time_us for k in self.kernels) or 1e-9
            name_w = min(62, max(len(k.name) for k in shown))
            out.append("  kernels by device time:")
            for k in shown:
                out.append(f"    {k.name[:name_w].ljust(name_w)}  "
                           f"{self._per_call(k.launches):>5.1f} launches  "
                           f"{self._per_call(k.device_time_us):>9.1f} us  "
                           f"{100.0 * k.device_time_us / total:>5.1f}%")
        if self.trace_path is not None:
            out.append(f"  chrome trace: {self.trace_path}")
        return "\n".join(out)


def _device_us(event) -> float:
    """Duration of one device-side event (a kernel execution), in microseconds."""
    return float(event.time_range.elapsed_us())


def _group(events: Iterable) -> tuple[KernelRecord, ...]:
    launches: dict[str, int] = defaultdict(int)
    busy: dict[str, float] = defaultdict(float)
    for ev in events:
        if ev.device_type != DeviceType.CUDA:
            continue
        us = _device_us(ev)
        if us <= 0:
            continue
        launches[ev.name] += 1
        busy[ev.name] += us
    records = (KernelRecord(n, launches[n], busy[n]) for n in launches)
    return tuple(sorted(records, key=lambda r: (-r.device_time_us, r.name)))


def profile_kernels(
    fn: Callable[[], object],
    *,
    label: str,
    warmup: int = 10,
    iterations: int = 20,
    trace_path: str | Path | None = None,
) -> ProfileResult:
    """Run ``fn`` ``iterations`` times under the profiler and group its device kernels."""
    if not torch.cuda.is_available():
        raise RuntimeError("kernel attribution needs a ROCm device")
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    wanted = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    with torch.profiler.profile(activities=wanted) as prof:
        for _ in range(iterations):
            fn()
        torch.cuda.synchronize()
    saved = None
    if trace_path is not None:
        saved = Path(trace_path)
        saved.parent.mkdir(parents=True, exist_ok=True)
        prof.export_chrome_trace(str(saved))
    return ProfileResult(label, iterations, _group(prof.events()), saved)


def launches_per_iteration(fn: Callable[[], object], *, warmup: int = 3,
                           iterations: int = 5) -> float:
    """Device kernels one call of ``fn`` launches, on average."""
    return profile_kernels(fn, label="", warmup=warmup, iterations=iterations).launches_per_iteration


def compare_launch_counts(candidates: dict[str, Callable[[], object]], *, warmup: int = 10,
                          iterations: int = 20) -> list[ProfileResult]:
    """:func:`profile_kernels` for each labelled implementation, in order."""
    return [profile_kernels(fn, label=label, warmup=warmup, iterations=iterations)
            for label, fn in candidates.items()]
