"""Profiling: kernel attribution (torch.profiler) and rocprofv3 summaries."""

from kernelforge.profiling.launches import (
    KernelRecord,
    ProfileResult,
    compare_launch_counts,
    launches_per_iteration,
    profile_kernels,
)

__all__ = [
    "KernelRecord",
    "ProfileResult",
    "compare_launch_counts",
    "launches_per_iteration",
    "profile_kernels",
]
