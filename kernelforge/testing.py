"""The correctness gate every tuning candidate passes before it is timed.

Semantics are the reference's (kernelforge/testing.py:26-175), because they
define parity:

    error = max|out - ref| / max|ref|       (max|out - ref| when ref is all zero)

passes at or below one threshold per dtype -- fp32 1e-5, fp16 5e-3,
bf16 2e-2. A shape mismatch or any non-finite output fails with an infinite
error; an empty tensor passes. The comparison runs in fp32.

The implementation is built for a device-resident output: every statistic the
verdict needs (non-finite count, largest difference, reference scale, and the
count of elements beyond the budget) is reduced on the output's device and
fetched with one host synchronisation, instead of one per statistic.
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass

import torch

ERROR_THRESHOLDS: dict[torch.dtype, float] = {
    torch.float32: 1e-5,
    torch.float16: 5e-3,
    torch.bfloat16: 2e-2,
}


@dataclass(frozen=True)
class VerificationResult:
    passed: bool
    error: float
    max_abs_err: float
    mismatched: int
    total: int
    threshold: float
    reason: str = ""

    def __str__(self) -> str:
        if not self.passed:
            return f"FAIL ({self.reason})"
        return f"ok (err={self.error:.3e} <= {self.threshold:.1e})"


def threshold_for(dtype: torch.dtype) -> float:
    if dtype in ERROR_THRESHOLDS:
        return ERROR_THRESHOLDS[dtype]
    known = sorted(str(d) for d in ERROR_THRESHOLDS)
    raise ValueError(f"no correctness threshold defined for {dtype}; known dtypes: {known}")


class Gate:
    """A normalised infinity-norm check at one threshold."""

    def __init__(self, threshold: float) -> None:
        self.threshold = float(threshold)

    @classmethod
    def for_dtype(cls, dtype: torch.dtype) -> Gate:
        return cls(threshold_for(dtype))

    def _fail(self, total: int, bad: int, reason: str) -> VerificationResult:
        inf = float("inf")
        return VerificationResult(False, inf, inf, bad, total, self.threshold, reason)

    def check(self, reference: torch.Tensor, output: torch.Tensor) -> VerificationResult:
        total = output.numel()
        if tuple(reference.shape) != tuple(output.shape):
            return self._fail(total, total, f"shape mismatch: reference {tuple(reference.shape)} "
                                            f"vs output {tuple(output.shape)}")
        if total == 0:
            return VerificationResult(True, 0.0, 0.0, 0, 0, self.threshold)

        out = output.detach().float()
        ref = reference.detach().to(device=out.device, dtype=torch.float32)
        diff = (out - ref).abs()
        scale = ref.abs().max()
        # Elements beyond the same bound the verdict uses, so a failing check
        # never reports that nothing differs.
        budget = torch.where(scale > 0, scale * self.threshold,
                             torch.full_like(scale, self.threshold))
        stats = torch.stack([
            (~torch.isfinite(out)).sum().float(),
            diff.max(),
            scale,
            (diff > budget).sum().float(),
        ]).tolist()  # the one synchronisation
        non_finite, max_abs, ref_scale, beyond = stats
        if non_finite:
            bad = int(non_finite)
            return self._fail(total, bad, f"output contains {bad}/{total} non-finite values")
        error = max_abs / ref_scale if ref_scale > 0 else max_abs
        ok = error <= self.threshold
        reason = "" if ok else (
            f"normalised error {error:.3e} exceeds {self.threshold:.1e} "
            f"(max|diff|={max_abs:.3e}, {int(beyond)}/{total} elements off)"
        )
        return VerificationResult(ok, error, max_abs, int(beyond), total, self.threshold, reason)


def verify(
    reference: torch.Tensor,
    output: torch.Tensor,
    *,
    dtype: torch.dtype | None = None,
    threshold: float | None = None,
) -> VerificationResult:
    """Gate ``output`` against ``reference``.

    ``dtype`` picks the threshold (default: the output's dtype); pass it when
    the reference was computed at higher precision than the kernel. The
    reference may live on another device; it is moved to the output's.
    """
    gate = Gate(threshold) if threshold is not None else Gate.for_dtype(dtype or output.dtype)
    return gate.check(reference, output)


def assert_verified(
    reference: torch.Tensor,
    output: torch.Tensor,
    *,
    dtype: torch.dtype | None = None,
    threshold: float | None = None,
    context: str = "",
) -> VerificationResult:
    """:func:`verify`, raising ``AssertionError`` (prefixed by ``context``) on failure."""
    result = verify(reference, output, dtype=dtype, threshold=threshold)
    if result.passed:
        return result
    raise AssertionError(f"{context}: {result.reason}" if context else result.reason)


@contextlib.contextmanager
def exact_fp32_matmul():
    """Run fp32 matmuls at full fp32 precision inside the block.

    A reduced-precision (TF32/XF32) fp32 product carries about 1e-3 relative
    error, a hundred times the fp32 threshold, so an fp32 reference computed
    that way would be the least accurate number in the comparison. On ROCm
    the same torch switches govern hipBLASLt; on the CPU they are inert.
    """
    saved = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32,
             torch.get_float32_matmul_precision())
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    try:
        yield
    finally:
        torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32 = saved[:2]
        torch.set_float32_matmul_precision(saved[2])
