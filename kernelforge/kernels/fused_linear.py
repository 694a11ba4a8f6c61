"""Fused linear + bias + tanh-GELU: ``y = gelu(x @ w + bias)`` in one launch.

Python surface of the reference's ``fused_linear_gelu``
(kernelforge/kernels/fused_linear.py:112-216). The bias is added to the fp32
accumulator and the activation applied while the tile is still in registers:

    gelu(a) = a / (1 + exp(-2*sqrt(2/pi) * (a + 0.044715 a^3)))

(the tanh form rewritten through ``tanh z = 2 sigmoid(2z) - 1``, one exp per
element, fused_linear.py:15-25). Unfused that is three launches and ``5*M*N``
of output traffic; fused, one launch and ``M*N``.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from kernelforge.benchmark import metrics
from kernelforge.kernels.base import Operator, cpu_generator
from kernelforge.kernels.matmul import _heuristic_config, default_gemm_config, launch_gemm
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import FusedLinearSearchSpace

#: 2*sqrt(2/pi), the sigmoid identity's factor of two folded in (fused_linear.py:46).
GELU_COEFF = 1.5957691216057308

DEFAULT_CONFIG = KernelConfig(
    "fused_linear", BLOCK_M=128, BLOCK_N=128, BLOCK_K=64, GROUP_M=8, num_warps=4, num_stages=2
)


def fused_linear_gelu(
    x: torch.Tensor,
    w: torch.Tensor,
    bias: torch.Tensor,
    *,
    config: KernelConfig | None = None,
) -> torch.Tensor:
    """``gelu(x @ w + bias)`` in one kernel.

    ``w`` is ``(K, N)`` like ``torch.matmul``; an ``nn.Linear`` weight is
    passed as ``weight.t()`` and read through its strides, without a copy.
    """
    if x.ndim != 2 or w.ndim != 2:
        raise ValueError(f"expected 2D x and w, got {tuple(x.shape)} and {tuple(w.shape)}")
    if x.shape[1] != w.shape[0]:
        raise ValueError(f"shape mismatch: {tuple(x.shape)} @ {tuple(w.shape)}")
    if tuple(bias.shape) != (w.shape[1],):
        raise ValueError(f"bias must have shape ({w.shape[1]},), got {tuple(bias.shape)}")
    if not (x.dtype == w.dtype == bias.dtype):
        raise ValueError(f"dtype mismatch: {x.dtype}, {w.dtype}, {bias.dtype}")
    m, n = x.shape[0], w.shape[1]
    cfg = config or default_gemm_config("fused_linear", x, w)
    y = torch.empty((m, n), device=x.device, dtype=x.dtype)
    return launch_gemm(x, w, bias, y, cfg)


def linear_gelu_reference(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """The unfused sequence as a model would write it (fused_linear.py:160-162)."""
    return torch.nn.functional.gelu(torch.matmul(x, w) + bias, approximate="tanh")


class FusedLinearOperator(Operator):
    name = "fused_linear"
    config_order = (
        "BLOCK_M", "BLOCK_N", "BLOCK_K", "GROUP_M", "DIRECT", "GEMV", "SPLIT_K", "num_warps",
        "num_stages",
    )

    def search_space(self) -> FusedLinearSearchSpace:
        return FusedLinearSearchSpace()

    def make_inputs(
        self, problem: Problem, device: torch.device, *, seed: int = 0
    ) -> tuple[torch.Tensor, ...]:
        gen = cpu_generator(seed)
        d = problem.dims_dict
        x = torch.randn(d["M"], d["K"], dtype=problem.dtype, generator=gen)
        # Scaled like an initialised weight so the pre-activation lands where
        # GELU is nonlinear (fused_linear.py:179-183).
        w = torch.randn(d["K"], d["N"], dtype=torch.float32, generator=gen)
        w = (w * (d["K"] ** -0.5)).to(problem.dtype)
        bias = torch.randn(d["N"], dtype=problem.dtype, generator=gen)
        if problem.layout == "bt":  # an nn.Linear weight passed as weight.t()
            return x.to(device), w.t().contiguous().to(device).t(), bias.to(device)
        return x.to(device), w.to(device), bias.to(device)

    def reference(self, *inputs: torch.Tensor) -> torch.Tensor:
        x, w, bias = inputs
        return linear_gelu_reference(x, w, bias)

    def availability(self, config: KernelConfig, problem: Problem) -> str:
        from kernelforge.kernels.matmul import gemm_availability

        return gemm_availability(config, problem.dtype)

    def run(self, config: KernelConfig, *inputs: torch.Tensor) -> torch.Tensor:
        x, w, bias = inputs
        return fused_linear_gelu(x, w, bias, config=config)

    def default_config(self, problem: Problem) -> KernelConfig:
        d = problem.dims_dict
        return _heuristic_config("fused_linear", d["M"], d["N"], d["K"], problem.dtype, problem.layout)

    def flops(self, problem: Problem) -> int:
        d = problem.dims_dict
        return metrics.matmul_flops(d["M"], d["N"], d["K"])

    def bytes_moved(self, problem: Problem) -> int:
        d = problem.dims_dict
        return metrics.fused_linear_bytes(d["M"], d["N"], d["K"], problem.itemsize, fused=True)

    def baselines(
        self, problem: Problem, inputs: tuple[torch.Tensor, ...]
    ) -> dict[str, Callable[[], torch.Tensor]]:
        x, w, bias = inputs
        return {
            "torch_eager": lambda: linear_gelu_reference(x, w, bias),
            "hip_default": lambda: fused_linear_gelu(x, w, bias, config=DEFAULT_CONFIG),
        }
