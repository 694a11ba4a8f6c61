"""Correctness gate.

Every tuning candidate passes :func:`verify` before it may be timed, so an
incorrect configuration is never ranked. The metric is the reference's
scale-invariant normalised infinity norm (kernelforge/testing.py:64-139),

    err = max|out - ref| / max|ref|

with one threshold per dtype (fp32 1e-5, fp16 5e-3, bf16 2e-2), falling back
to the absolute error for an all-zero reference. Shape mismatch and
non-finite output fail with ``inf``; an empty tensor passes.
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
        if self.passed:
            return f"ok (err={self.error:.3e} <= {self.threshold:.1e})"
        return f"FAIL ({self.reason})"


def threshold_for(dtype: torch.dtype) -> float:
    try:
        return ERROR_THRESHOLDS[dtype]
    except KeyError:
        raise ValueError(
            f"no correctness threshold defined for {dtype}; "
            f"known dtypes: {sorted(str(d) for d in ERROR_THRESHOLDS)}"
        ) from None


def verify(
    reference: torch.Tensor,
    output: torch.Tensor,
    *,
    dtype: torch.dtype | None = None,
    threshold: float | None = None,
) -> VerificationResult:
    """Compare a kernel output against a reference.

    ``dtype`` selects the threshold and defaults to the output dtype. The
    comparison itself runs in fp32 on the output's device; a reference on
    another device is moved there.
    """
    gate_dtype = dtype if dtype is not None else output.dtype
    limit = threshold if threshold is not None else threshold_for(gate_dtype)

    if tuple(reference.shape) != tuple(output.shape):
        return VerificationResult(
            passed=False,
            error=float("inf"),
            max_abs_err=float("inf"),
            mismatched=output.numel(),
            total=output.numel(),
            threshold=limit,
            reason=(
                f"shape mismatch: reference {tuple(reference.shape)} vs output "
                f"{tuple(output.shape)}"
            ),
        )

    out = output.detach().to(torch.float32)
    ref = reference.detach().to(device=out.device, dtype=torch.float32)
    total = out.numel()
    if total == 0:
        return VerificationResult(True, 0.0, 0.0, 0, 0, limit)

    finite = torch.isfinite(out)
    if not bool(finite.all()):
        n_bad = int((~finite).sum())
        return VerificationResult(
            passed=False,
            error=float("inf"),
            max_abs_err=float("inf"),
            mismatched=n_bad,
            total=total,
            threshold=limit,
            reason=f"output contains {n_bad}/{total} non-finite values",
        )

    diff = (out - ref).abs()
    max_abs_err = float(diff.max())
    scale = float(ref.abs().max())
    error = max_abs_err / scale if scale > 0 else max_abs_err
    passed = error <= limit
    budget = limit * scale if scale > 0 else limit
    mismatched = int((diff > budget).sum())
    return VerificationResult(
        passed=passed,
        error=error,
        max_abs_err=max_abs_err,
        mismatched=mismatched,
        total=total,
        threshold=limit,
        reason=(
            ""
            if passed
            else (
                f"normalised error {error:.3e} exceeds {limit:.1e} "
                f"(max|diff|={max_abs_err:.3e}, {mismatched}/{total} elements off)"
            )
        ),
    )


def assert_verified(
    reference: torch.Tensor,
    output: torch.Tensor,
    *,
    dtype: torch.dtype | None = None,
    threshold: float | None = None,
    context: str = "",
) -> VerificationResult:
    result = verify(reference, output, dtype=dtype, threshold=threshold)
    if not result.passed:
        prefix = f"{context}: " if context else ""
        raise AssertionError(f"{prefix}{result.reason}")
    return result


@contextlib.contextmanager
def exact_fp32_matmul():
    """Disable reduced-precision fp32 matmuls for the duration of the block.

    An fp32 reference must be computed at full fp32 precision or it is the
    least accurate number in the comparison (testing.py:157-175). On ROCm the
    same torch flags govern hipBLASLt's TF32/XF32 paths; the CPU ignores them.
    """
    prev_matmul = torch.backends.cuda.matmul.allow_tf32
    prev_cudnn = torch.backends.cudnn.allow_tf32
    prev_precision = torch.get_float32_matmul_precision()
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    try:
        yield
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev_matmul
        torch.backends.cudnn.allow_tf32 = prev_cudnn
        torch.set_float32_matmul_precision(prev_precision)
