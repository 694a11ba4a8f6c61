"""Single-pass row softmax on gfx950.

Python surface of the reference's ``softmax`` (kernelforge/kernels/softmax.py:
61-157): 2-D input with a contiguous last dimension, fp32 internal max/sum,
output in the input dtype. Subtracting the row max first is required, not an
optimisation: fp16 ``exp`` overflows above ~11 (softmax.py:1-15).

One workgroup reads each row exactly once into registers (16-byte loads),
reduces max and sum with wave64 shuffles plus one LDS exchange, and writes
the row once.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from kernelforge.benchmark import metrics
from kernelforge.dtypes import abi_code
from kernelforge.kernels.base import Operator, cpu_generator
from kernelforge.runtime import hip
from kernelforge.runtime.dispatch import shipped_config
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import SoftmaxSearchSpace, default_row_config


def default_config(n_cols: int) -> KernelConfig:
    return default_row_config("softmax", n_cols)


def _check_row_config(cfg: KernelConfig, n_cols: int, limit: int, what: str) -> None:
    block = cfg["BLOCK_SIZE"]
    if block < n_cols:
        raise ValueError(
            f"BLOCK_SIZE={block} cannot hold a row of {n_cols}; "
            "this kernel is single-pass by design"
        )
    if block > limit:
        raise ValueError(f"{what} {n_cols} exceeds the single-pass limit of {limit}")


def softmax(x: torch.Tensor, *, config: KernelConfig | None = None) -> torch.Tensor:
    if x.ndim != 2:
        raise ValueError(f"expected a 2D tensor, got shape {tuple(x.shape)}")
    if x.stride(1) != 1 and x.shape[1] > 1:
        raise ValueError(
            "x must have a contiguous last dimension; this kernel indexes columns "
            "directly off the row pointer. Pass x.contiguous() -- explicitly, so the "
            "copy is not hidden inside a measured region."
        )
    n_rows, n_cols = x.shape
    cfg = (config or shipped_config("softmax", x.dtype, x.device, rows=n_rows, cols=n_cols)
           or default_config(n_cols))
    _check_row_config(cfg, n_cols, SoftmaxSearchSpace.MAX_BLOCK_SIZE, "row width")
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    hip.require_device_tensor(x)
    lib = hip.load()
    rc = lib.kf_softmax(
        abi_code(x.dtype), x.data_ptr(), out.data_ptr(), n_rows, n_cols,
        x.stride(0) if n_rows > 1 else n_cols, out.stride(0) if n_rows > 1 else n_cols,
        cfg["BLOCK_SIZE"], cfg["ROWS_PER_PROGRAM"], cfg["num_warps"], hip.stream_of(x),
    )
    hip.check(rc, "softmax")
    return out


class SoftmaxOperator(Operator):
    name = "softmax"
    config_order = ("BLOCK_SIZE", "ROWS_PER_PROGRAM", "num_warps")

    def search_space(self) -> SoftmaxSearchSpace:
        return SoftmaxSearchSpace()

    def make_inputs(
        self, problem: Problem, device: torch.device, *, seed: int = 0
    ) -> tuple[torch.Tensor, ...]:
        gen = cpu_generator(seed)
        d = problem.dims_dict
        x = torch.randn(d["rows"], d["cols"], dtype=problem.dtype, generator=gen)
        return (x.to(device),)

    def reference(self, *inputs: torch.Tensor) -> torch.Tensor:
        (x,) = inputs
        return torch.softmax(x, dim=-1)

    def run(self, config: KernelConfig, *inputs: torch.Tensor) -> torch.Tensor:
        (x,) = inputs
        return softmax(x, config=config)

    def default_config(self, problem: Problem) -> KernelConfig:
        return default_config(problem.dims_dict["cols"])

    def flops(self, problem: Problem) -> int:
        d = problem.dims_dict
        # max, subtract, exp, sum, divide: an approximation; GB/s is the metric.
        return 5 * d["rows"] * d["cols"]

    def bytes_moved(self, problem: Problem) -> int:
        d = problem.dims_dict
        return metrics.softmax_bytes(d["rows"], d["cols"], problem.itemsize)

    def is_memory_bound(self) -> bool:
        return True

    def baselines(
        self, problem: Problem, inputs: tuple[torch.Tensor, ...]
    ) -> dict[str, Callable[[], torch.Tensor]]:
        (x,) = inputs
        cols = problem.dims_dict["cols"]
        return {
            "torch_eager": lambda: torch.softmax(x, dim=-1),
            "hip_default": lambda: softmax(x, config=default_config(cols)),
        }
