"""A pre-norm decoder block whose norms and MLP activation run on kernelforge.

The dispatch consumer of the reference (kernelforge/integration/
transformer.py:71-187): the first caller that takes its kernel configurations
from the winner cache rather than from a tuning run. What it shows is
Amdahl's law at block scale: the two RMSNorms and the MLP up-projection with
its bias + GELU are swapped for this package's kernels, while attention
(``scaled_dot_product_attention``) and the QKV, output and down projections
stay on PyTorch, so the block-level speedup is bounded by the share of block
time the swapped operators held.

``backend`` is a mutable attribute of one module, so both backends run on the
same weights and a difference in output can only come from the kernels.

On MI355X the swapped MLP up-projection takes the direct-to-LDS MFMA GEMM
with the fused epilogue for prefill rows and the split-K GEMV (same
epilogue) for decode rows (M <= 8), whichever the cached or packaged winner
names; ``mlp_up.weight.t()`` is consumed through its strides (B k-contiguous),
so no transposed copy is made.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from kernelforge.kernels.fused_linear import fused_linear_gelu
from kernelforge.kernels.rmsnorm import DEFAULT_EPS, rmsnorm, rmsnorm_reference
from kernelforge.runtime.dispatch import select_config
from kernelforge.tuning.cache import ConfigCache
from kernelforge.tuning.config import KernelConfig, Problem

BACKEND_TORCH = "torch"
BACKEND_KERNELO = "kernelforge"
BACKENDS = (BACKEND_TORCH, BACKEND_KERNELO)


@dataclass(frozen=True)
class BlockConfig:
    """Geometry of one block; the default is Llama-2-7B's (4096 hidden, 32
    heads, 11008 intermediate). The MLP is GELU rather than SwiGLU because the
    fused kernel's epilogue is bias + GELU; the matrix shapes are the real ones."""

    hidden: int = 4096
    heads: int = 32
    intermediate: int = 11008
    eps: float = DEFAULT_EPS

    def __post_init__(self) -> None:
        if self.hidden % self.heads:
            raise ValueError(f"hidden {self.hidden} is not divisible by {self.heads} heads")

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


class TransformerBlock(nn.Module):
    """Pre-norm decoder block with swappable normalisation and MLP activation."""

    def __init__(
        self,
        config: BlockConfig | None = None,
        *,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str = "cuda",
        backend: str = BACKEND_TORCH,
        cache: ConfigCache | None = None,
    ) -> None:
        super().__init__()
        if backend not in BACKENDS:
            raise ValueError(f"backend must be one of {BACKENDS}, got {backend!r}")
        self.config = config or BlockConfig()
        self.backend = backend
        self._cache = cache
        # Selection reads the cache files; it runs once per (operation, shape).
        self._selected: dict[tuple[str, int, int], KernelConfig] = {}

        hidden, intermediate = self.config.hidden, self.config.intermediate
        factory = {"device": device, "dtype": dtype}
        self.attn_norm_weight = nn.Parameter(torch.ones(hidden, **factory))
        self.mlp_norm_weight = nn.Parameter(torch.ones(hidden, **factory))
        self.qkv_proj = nn.Linear(hidden, 3 * hidden, bias=False, **factory)
        self.out_proj = nn.Linear(hidden, hidden, bias=False, **factory)
        self.mlp_up = nn.Linear(hidden, intermediate, bias=True, **factory)
        self.mlp_down = nn.Linear(intermediate, hidden, bias=False, **factory)

    def _config_for(self, operation: str, rows: int, cols: int, dtype: torch.dtype) -> KernelConfig:
        key = (operation, rows, cols)
        cfg = self._selected.get(key)
        if cfg is None:
            from kernelforge.kernels import get_operator

            if operation == "rmsnorm":
                problem = Problem.create(operation, dtype, rows=rows, cols=cols)
            else:
                problem = Problem.create(operation, dtype, M=rows, N=self.config.intermediate, K=cols)
            cfg = select_config(get_operator(operation), problem, cache=self._cache).config
            self._selected[key] = cfg
        return cfg

    def _norm(self, flat: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        if self.backend == BACKEND_TORCH:
            return rmsnorm_reference(flat, weight, eps=self.config.eps)
        cfg = self._config_for("rmsnorm", flat.shape[0], flat.shape[1], flat.dtype)
        return rmsnorm(flat, weight, eps=self.config.eps, config=cfg)

    def _mlp_activation(self, flat: torch.Tensor) -> torch.Tensor:
        if self.backend == BACKEND_TORCH:
            return F.gelu(self.mlp_up(flat), approximate="tanh")
        cfg = self._config_for("fused_linear", flat.shape[0], flat.shape[1], flat.dtype)
        return fused_linear_gelu(flat, self.mlp_up.weight.t(), self.mlp_up.bias, config=cfg)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.ndim != 3:
            raise ValueError(f"expected (batch, seq, hidden), got {tuple(x.shape)}")
        batch, seq, hidden = x.shape
        if hidden != self.config.hidden:
            raise ValueError(f"expected hidden {self.config.hidden}, got {hidden}")
        heads, head_dim = self.config.heads, self.config.head_dim
        tokens = batch * seq

        normed = self._norm(x.reshape(tokens, hidden), self.attn_norm_weight)
        qkv = self.qkv_proj(normed).view(batch, seq, 3, heads, head_dim)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        attended = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + self.out_proj(attended.transpose(1, 2).reshape(batch, seq, hidden))

        normed = self._norm(x.reshape(tokens, hidden), self.mlp_norm_weight)
        return x + self.mlp_down(self._mlp_activation(normed)).view(batch, seq, hidden)


def benchmark_block(
    config: BlockConfig | None = None,
    *,
    batch: int = 1,
    seq: int = 2048,
    dtype: torch.dtype = torch.float16,
    device: torch.device | str = "cuda",
    warmup: int = 25,
    iterations: int = 100,
    cache: ConfigCache | None = None,
) -> dict[str, object]:
    """Time one block per backend on identical weights and inputs.

    No cache flush between iterations (transformer.py:176-186 in the
    reference): a block's working set (about 300 MiB of fp16 weights at the
    default geometry) is larger than L2 plus the Infinity Cache anyway.
    """
    from kernelforge.benchmark.runner import benchmark

    block = TransformerBlock(config, dtype=dtype, device=device, cache=cache)
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(batch, seq, block.config.hidden, generator=gen).to(device=device, dtype=dtype)
    results: dict[str, object] = {}
    with torch.inference_mode():
        for backend in BACKENDS:
            block.backend = backend
            results[backend] = benchmark(
                lambda: block(x), warmup=warmup, iterations=iterations, device=device,
                flush_l2=False,
            )
    return results
