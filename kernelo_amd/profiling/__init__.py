"""Profiling: kernel attribution (torch.profiler) and rocprofv3 summaries."""

from kernelo_amd.profiling.launches import (
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
