"""Derived performance metrics: FLOP and minimum-byte models, roofline helpers.

The byte counts are minimum traffic -- each input read once, each output
written once -- as in the reference (kernelforge/benchmark/metrics.py:17-88).
"""

from __future__ import annotations


def matmul_flops(m: int, n: int, k: int) -> int:
    """``2*M*N*K``."""
    return 2 * m * n * k


def matmul_bytes(m: int, n: int, k: int, itemsize: int) -> int:
    """Read A and B once, write C once."""
    return (m * k + k * n + m * n) * itemsize


def elementwise_bytes(elements: int, itemsize: int, *, tensors: int) -> int:
    return elements * itemsize * tensors


def vector_add_bytes(n: int, itemsize: int) -> int:
    """Read a and b, write c."""
    return elementwise_bytes(n, itemsize, tensors=3)


def rmsnorm_bytes(rows: int, cols: int, itemsize: int) -> int:
    """Read x, write y, read gamma once per launch."""
    return (2 * rows * cols + cols) * itemsize


def softmax_bytes(rows: int, cols: int, itemsize: int) -> int:
    """Read x once, write y once."""
    return elementwise_bytes(rows * cols, itemsize, tensors=2)


def fused_linear_bytes(m: int, n: int, k: int, itemsize: int, *, fused: bool) -> int:
    """``gelu(x @ w + bias)``: ``M*N`` output traffic fused, ``5*M*N`` unfused."""
    operands = m * k + k * n + n
    output = m * n if fused else 5 * m * n
    return (operands + output) * itemsize


def tflops(flops: int, ms: float) -> float:
    if ms <= 0:
        raise ValueError(f"latency must be positive, got {ms}")
    return flops / (ms * 1e-3) / 1e12


def gbps(num_bytes: int, ms: float) -> float:
    if ms <= 0:
        raise ValueError(f"latency must be positive, got {ms}")
    return num_bytes / (ms * 1e-3) / 1e9


def arithmetic_intensity(flops: int, num_bytes: int) -> float:
    """FLOP per byte. MI355X's ridge is 2516.6 TFLOP/s / 8 TB/s ~ 315 FLOP/B."""
    if num_bytes <= 0:
        raise ValueError(f"byte count must be positive, got {num_bytes}")
    return flops / num_bytes


def speedup(baseline_ms: float, candidate_ms: float) -> float:
    if candidate_ms <= 0:
        raise ValueError(f"latency must be positive, got {candidate_ms}")
    return baseline_ms / candidate_ms


def roofline_fraction(achieved: float, peak: float) -> float:
    if peak <= 0:
        raise ValueError(f"peak must be positive, got {peak}")
    return achieved / peak
