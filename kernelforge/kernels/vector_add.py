"""Elementwise ``c = a + b`` on gfx950: the pure HBM stream.

Python surface of the reference's ``vector_add`` (kernelforge/kernels/
vector_add.py:43-107): same signature and validation messages, contiguous
operands, output in the input dtype. The reference keeps it as the smallest
kernel that exercises the whole pipeline (search space, gate, timing,
database) and as a bandwidth probe against the spec sheet; here it is the
HBM sanity probe for MI355X (8 TB/s peak). One call into
``kf_vector_add``; the sum is formed in fp32 and rounded once, which for
16-bit inputs is exactly the correctly rounded 16-bit sum, so the result is
bit-identical to torch's ``a + b``.
"""

from __future__ import annotations

from collections.abc import Callable
from functools import lru_cache

import torch

from kernelforge.benchmark import metrics
from kernelforge.dtypes import abi_code
from kernelforge.kernels.base import Operator, cpu_generator
from kernelforge.runtime import hip
from kernelforge.runtime.env import MI355X_CAPS
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import VectorAddSearchSpace

#: The fixed configuration the tuned one is compared against
#: (vector_add.py:43 in the reference).
DEFAULT_CONFIG = KernelConfig("vector_add", BLOCK_SIZE=1024, num_warps=4)


@lru_cache(maxsize=256)
def _heuristic_config(n: int, dtype: torch.dtype) -> KernelConfig:
    """The search space's top-priority candidate for the MI355X model."""
    problem = Problem.create("vector_add", dtype, n=max(n, 1))
    best = VectorAddSearchSpace().candidates(problem, MI355X_CAPS, max_candidates=1)
    return best[0] if best else DEFAULT_CONFIG


def vector_add(
    a: torch.Tensor, b: torch.Tensor, *, config: KernelConfig | None = None
) -> torch.Tensor:
    if a.shape != b.shape:
        raise ValueError(f"shape mismatch: {tuple(a.shape)} vs {tuple(b.shape)}")
    if a.dtype != b.dtype:
        raise ValueError(f"dtype mismatch: {a.dtype} vs {b.dtype}")
    cfg = config or DEFAULT_CONFIG
    a, b = a.contiguous(), b.contiguous()
    out = torch.empty_like(a, memory_format=torch.contiguous_format)
    hip.require_device_tensor(a, b)
    lib = hip.load()
    rc = lib.kf_vector_add(
        abi_code(a.dtype), a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(),
        cfg["BLOCK_SIZE"], cfg["num_warps"], hip.stream_of(a),
    )
    hip.check(rc, "vector_add")
    return out


class VectorAddOperator(Operator):
    name = "vector_add"
    config_order = ("BLOCK_SIZE", "num_warps")

    def search_space(self) -> VectorAddSearchSpace:
        return VectorAddSearchSpace()

    def make_inputs(
        self, problem: Problem, device: torch.device, *, seed: int = 0
    ) -> tuple[torch.Tensor, ...]:
        gen = cpu_generator(seed)
        n = problem.dims_dict["n"]
        a = torch.randn(n, dtype=problem.dtype, generator=gen)
        b = torch.randn(n, dtype=problem.dtype, generator=gen)
        return a.to(device), b.to(device)

    def reference(self, *inputs: torch.Tensor) -> torch.Tensor:
        a, b = inputs
        return a + b

    def run(self, config: KernelConfig, *inputs: torch.Tensor) -> torch.Tensor:
        a, b = inputs
        return vector_add(a, b, config=config)

    def default_config(self, problem: Problem) -> KernelConfig:
        return _heuristic_config(problem.dims_dict["n"], problem.dtype)

    def flops(self, problem: Problem) -> int:
        return problem.dims_dict["n"]

    def bytes_moved(self, problem: Problem) -> int:
        return metrics.vector_add_bytes(problem.dims_dict["n"], problem.itemsize)

    def is_memory_bound(self) -> bool:
        return True

    def baselines(
        self, problem: Problem, inputs: tuple[torch.Tensor, ...]
    ) -> dict[str, Callable[[], torch.Tensor]]:
        a, b = inputs
        return {
            "torch_eager": lambda: a + b,
            "hip_default": lambda: vector_add(a, b, config=DEFAULT_CONFIG),
        }
