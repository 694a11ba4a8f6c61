"""Kernel attribution with ``torch.profiler`` (launches per call, device time per kernel).

The latency harness says how long; this says *what ran*. For the fusion
comparison the launch count is the evidence: the unfused sequence launches
at least three kernels per call, the fused one exactly one
(kernelforge/profiling/pytorch_profiler.py:53-60,91-135). On ROCm the
profiler's device activity comes from the HIP runtime, so launches made
through ``libkernelforge_hip.so`` are attributed like torch's own.

Tracing perturbs timing: these figures are for attribution, not headline
latency (that comes from the hipEvent harness).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch
from torch.autograd import DeviceType


def _device_time_us(event) -> float:
    for attribute in ("device_time_total", "cuda_time_total"):
        value = getattr(event, attribute, None)
        if value is not None:
            return float(value)
    return 0.0


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

    @property
    def launches_per_iteration(self) -> float:
        total = sum(k.launches for k in self.kernels)
        return total / self.iterations if self.iterations else 0.0

    @property
    def device_time_per_iteration_us(self) -> float:
        total = sum(k.device_time_us for k in self.kernels)
        return total / self.iterations if self.iterations else 0.0

    def render(self, limit: int = 10) -> str:
        lines = [
            self.label,
            f"  kernel launches per call : {self.launches_per_iteration:.2f}",
            f"  device time per call     : {self.device_time_per_iteration_us:.1f} us",
        ]
        if self.kernels:
            total = max(sum(k.device_time_us for k in self.kernels), 1e-9)
            width = min(62, max(len(k.name) for k in self.kernels))
            lines.append("  kernels by device time:")
            for k in self.kernels[:limit]:
                lines.append(
                    f"    {k.name[:width]:<{width}}  "
                    f"{k.launches / max(self.iterations, 1):>5.1f} launches  "
                    f"{k.device_time_us / max(self.iterations, 1):>9.1f} us  "
                    f"{k.device_time_us / total * 100:>5.1f}%"
                )
        if self.trace_path is not None:
            lines.append(f"  chrome trace: {self.trace_path}")
        return "\n".join(lines)


def profile_kernels(
    fn,
    *,
    label: str,
    warmup: int = 10,
    iterations: int = 20,
    trace_path: str | Path | None = None,
) -> ProfileResult:
    """Profile ``fn`` and attribute device time to individual kernels."""
    if not torch.cuda.is_available():
        raise RuntimeError("kernel attribution needs a ROCm device")
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    activities = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    with torch.profiler.profile(activities=activities) as prof:
        for _ in range(iterations):
            fn()
        torch.cuda.synchronize()
    kernels = [
        KernelRecord(name=e.key, launches=int(e.count), device_time_us=_device_time_us(e))
        for e in prof.key_averages()
        if e.device_type == DeviceType.CUDA and _device_time_us(e) > 0
    ]
    kernels.sort(key=lambda k: -k.device_time_us)
    resolved = None
    if trace_path is not None:
        resolved = Path(trace_path)
        resolved.parent.mkdir(parents=True, exist_ok=True)
        prof.export_chrome_trace(str(resolved))
    return ProfileResult(label=label, iterations=iterations, kernels=tuple(kernels), trace_path=resolved)


def launches_per_iteration(fn, *, warmup: int = 3, iterations: int = 5) -> float:
    return profile_kernels(fn, label="", warmup=warmup, iterations=iterations).launches_per_iteration


def compare_launch_counts(
    candidates: dict[str, object], *, warmup: int = 10, iterations: int = 20
) -> list[ProfileResult]:
    return [
        profile_kernels(fn, label=label, warmup=warmup, iterations=iterations)
        for label, fn in candidates.items()
    ]
