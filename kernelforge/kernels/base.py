"""The contract a tunable operator fulfils (kernelforge/kernels/base.py:21-78).

The tuner knows nothing about GEMMs: it asks an operator for a search space,
inputs, a reference result and a way to run one configuration. Filtering,
verification, timing, ranking and persistence are generic.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Callable

import torch

from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import SearchSpace


class Operator(ABC):
    """One tunable operation."""

    name: str
    #: Preferred key order when rendering a config in the CLI.
    config_order: tuple[str, ...] = ()

    @abstractmethod
    def search_space(self) -> SearchSpace: ...

    @abstractmethod
    def make_inputs(
        self, problem: Problem, device: torch.device, *, seed: int = 0
    ) -> tuple[torch.Tensor, ...]:
        """Reproducible inputs for ``problem`` on ``device``.

        Drawn on the CPU from ``torch.Generator().manual_seed(seed)`` and then
        copied, so a host-side oracle sees exactly the device's values.
        """

    @abstractmethod
    def reference(self, *inputs: torch.Tensor) -> torch.Tensor:
        """The PyTorch computation this kernel must agree with."""

    @abstractmethod
    def run(self, config: KernelConfig, *inputs: torch.Tensor) -> torch.Tensor:
        """Execute the HIP kernel with ``config``."""

    @abstractmethod
    def default_config(self, problem: Problem) -> KernelConfig:
        """A fixed, always-feasible configuration: the untuned baseline and
        the fallback when the cache misses."""

    @abstractmethod
    def flops(self, problem: Problem) -> int: ...

    @abstractmethod
    def bytes_moved(self, problem: Problem) -> int:
        """Minimum global-memory traffic in bytes (each input read once, each
        output written once)."""

    def baselines(
        self, problem: Problem, inputs: tuple[torch.Tensor, ...]
    ) -> dict[str, Callable[[], torch.Tensor]]:
        """Implementations to compare against, keyed by label.

        ``torch_eager`` (hipBLASLt / ATen-HIP on the GPU) is always present.
        """
        return {"torch_eager": lambda: self.reference(*inputs)}

    def availability(self, config: KernelConfig, problem: Problem) -> str:
        """Why ``config`` cannot run for ``problem`` in this build, or ``""``.

        Kernels are compiled ahead of time, so an operator can answer from
        the library's variant table without launching anything; the tuner
        records a non-empty answer as a compile error. The default claims
        every configuration is available and lets the launch decide.
        """
        return ""

    def is_memory_bound(self) -> bool:
        """Whether GB/s (True) or TFLOP/s (False) is the headline metric."""
        return False


def compiled_baseline(
    fn: Callable[..., torch.Tensor], inputs: tuple[torch.Tensor, ...], *, mode: str | None = None
) -> Callable[[], torch.Tensor]:
    """Wrap ``fn`` in ``torch.compile`` and warm it up once (base.py:80-94).

    Not part of any default baseline set here: on ROCm it lowers through
    Triton, which this build does not depend on. Callers may opt in.
    """
    compiled = torch.compile(fn, mode=mode) if mode else torch.compile(fn)

    def run() -> torch.Tensor:
        return compiled(*inputs)

    run()
    return run


def cpu_generator(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)
