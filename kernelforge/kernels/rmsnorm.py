"""RMSNorm on gfx950: ``y = x * rsqrt(mean(x^2) + eps) * gamma``.

Python surface of the reference's ``rmsnorm`` (kernelforge/kernels/rmsnorm.py:
38-206), which also replaces its handwritten CUDA kernel
(kernelforge/csrc/rmsnorm_kernel.cuh:38-88): the sum of squares, the rescale
and the gamma multiply are fp32 and the result is rounded once, so the fp16
sum-of-squares precision trap (rmsnorm.py:16-25) cannot occur. ``eps`` sits
inside the root, keeping an all-zero row finite.

Two kernels sit behind it. The single-pass kernel holds a row in registers
(up to 16384 values); a config with ``TWO_PASS=1`` selects the two-pass
kernel, which walks a row of any width twice, optionally parking it in LDS
in between (``STAGE_ROW=1``). The two-pass kernel is the reference's first
listed future improvement (README.md:656-660); the default configuration
uses it for rows beyond the single-pass limit.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from kernelforge.benchmark import metrics
from kernelforge.dtypes import abi_code
from kernelforge.kernels.base import Operator, cpu_generator
from kernelforge.kernels.softmax import _check_row_config
from kernelforge.runtime import hip
from kernelforge.runtime.dispatch import shipped_config
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import RMSNormSearchSpace, default_row_config

DEFAULT_EPS = 1e-5


def default_config(n_cols: int, dtype: torch.dtype | None = None) -> KernelConfig:
    return default_row_config("rmsnorm", n_cols, dtype)


def rmsnorm(
    x: torch.Tensor,
    gamma: torch.Tensor,
    *,
    eps: float = DEFAULT_EPS,
    config: KernelConfig | None = None,
) -> torch.Tensor:
    if x.ndim != 2:
        raise ValueError(f"expected a 2D tensor, got shape {tuple(x.shape)}")
    if x.stride(1) != 1 and x.shape[1] > 1:
        raise ValueError(
            "x must have a contiguous last dimension; this kernel indexes columns "
            "directly off the row pointer. Pass x.contiguous() -- explicitly, so the "
            "copy is not hidden inside a measured region."
        )
    n_rows, n_cols = x.shape
    if tuple(gamma.shape) != (n_cols,):
        raise ValueError(f"gamma must have shape ({n_cols},), got {tuple(gamma.shape)}")
    if gamma.stride(0) != 1 and n_cols > 1:
        raise ValueError("gamma must be contiguous")
    if gamma.dtype != x.dtype:
        raise ValueError(f"dtype mismatch: {x.dtype} vs {gamma.dtype}")
    cfg = (config or shipped_config("rmsnorm", x.dtype, x.device, rows=n_rows, cols=n_cols)
           or default_config(n_cols, x.dtype))
    if cfg.get("TWO_PASS"):
        return _rmsnorm_two_pass(x, gamma, float(eps), cfg)
    _check_row_config(cfg, n_cols, RMSNormSearchSpace.MAX_BLOCK_SIZE, "hidden size")
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    hip.require_device_tensor(x, gamma)
    lib = hip.load()
    rc = lib.kf_rmsnorm(
        abi_code(x.dtype), x.data_ptr(), gamma.data_ptr(), out.data_ptr(), n_rows, n_cols,
        x.stride(0) if n_rows > 1 else n_cols, out.stride(0) if n_rows > 1 else n_cols,
        float(eps), cfg["BLOCK_SIZE"], cfg["ROWS_PER_PROGRAM"], cfg["num_warps"],
        hip.stream_of(x),
    )
    hip.check(rc, "rmsnorm")
    return out


def _rmsnorm_two_pass(
    x: torch.Tensor, gamma: torch.Tensor, eps: float, cfg: KernelConfig
) -> torch.Tensor:
    n_rows, n_cols = x.shape
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    hip.require_device_tensor(x, gamma)
    lib = hip.load()
    rc = lib.kf_rmsnorm_two_pass(
        abi_code(x.dtype), x.data_ptr(), gamma.data_ptr(), out.data_ptr(), n_rows, n_cols,
        x.stride(0) if n_rows > 1 else n_cols, out.stride(0) if n_rows > 1 else n_cols,
        eps, cfg["BLOCK_SIZE"], cfg["ROWS_PER_PROGRAM"], cfg["num_warps"],
        int(cfg.get("STAGE_ROW", 0)), hip.stream_of(x),
    )
    hip.check(rc, "rmsnorm_two_pass")
    return out


def rmsnorm_reference(
    x: torch.Tensor, gamma: torch.Tensor, *, eps: float = DEFAULT_EPS
) -> torch.Tensor:
    """PyTorch RMSNorm with an fp32 reduction, rounded once (rmsnorm.py:130-143)."""
    xf = x.to(torch.float32)
    inv_rms = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * inv_rms * gamma.to(torch.float32)).to(x.dtype)


class RMSNormOperator(Operator):
    name = "rmsnorm"
    config_order = ("TWO_PASS", "BLOCK_SIZE", "ROWS_PER_PROGRAM", "STAGE_ROW", "num_warps")

    def __init__(self, eps: float = DEFAULT_EPS) -> None:
        self.eps = eps

    def search_space(self) -> RMSNormSearchSpace:
        return RMSNormSearchSpace()

    def make_inputs(
        self, problem: Problem, device: torch.device, *, seed: int = 0
    ) -> tuple[torch.Tensor, ...]:
        gen = cpu_generator(seed)
        d = problem.dims_dict
        x = torch.randn(d["rows"], d["cols"], dtype=problem.dtype, generator=gen)
        # gamma near 1, as after initialisation (rmsnorm.py:160-163).
        gamma = torch.randn(d["cols"], dtype=problem.dtype, generator=gen)
        gamma = (gamma * 0.1 + 1.0).to(problem.dtype)
        return x.to(device), gamma.to(device)

    def reference(self, *inputs: torch.Tensor) -> torch.Tensor:
        x, gamma = inputs
        return rmsnorm_reference(x, gamma, eps=self.eps)

    def run(self, config: KernelConfig, *inputs: torch.Tensor) -> torch.Tensor:
        x, gamma = inputs
        return rmsnorm(x, gamma, eps=self.eps, config=config)

    def default_config(self, problem: Problem) -> KernelConfig:
        return default_config(problem.dims_dict["cols"], problem.dtype)

    def flops(self, problem: Problem) -> int:
        d = problem.dims_dict
        return 4 * d["rows"] * d["cols"]

    def bytes_moved(self, problem: Problem) -> int:
        d = problem.dims_dict
        return metrics.rmsnorm_bytes(d["rows"], d["cols"], problem.itemsize)

    def is_memory_bound(self) -> bool:
        return True

    def baselines(
        self, problem: Problem, inputs: tuple[torch.Tensor, ...]
    ) -> dict[str, Callable[[], torch.Tensor]]:
        x, gamma = inputs
        cols = problem.dims_dict["cols"]
        return {
            "torch_eager": lambda: rmsnorm_reference(x, gamma, eps=self.eps),
            "hip_default": lambda: rmsnorm(
                x, gamma, eps=self.eps, config=default_config(cols, problem.dtype)
            ),
        }
