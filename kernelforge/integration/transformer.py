"""A pre-norm decoder block whose norms and MLP up-projection run on kernelforge.

The first consumer of the winner cache (kernelforge/integration/
transformer.py:71-187 plays the same role): it never tunes, it asks dispatch
for each kernel's configuration and runs it. It shows Amdahl's law at block
scale. Two operator paths implement the swappable pieces:

* ``torch``: RMSNorm as the reference formula, the MLP up-projection as
  ``nn.Linear`` followed by tanh-GELU (three launches);
* ``kernelforge``: the RMSNorm row kernel, and the up-projection with bias +
  GELU fused into one MFMA GEMM launch (the split-K GEMV at decode rows).

Attention (``scaled_dot_product_attention``) and the QKV, output and down
projections are PyTorch on both paths, so the block-level speedup is bounded
by the share of block time the swapped operators hold. ``backend`` is a
mutable attribute of one module: both paths run on the same weights, so a
difference in output can only come from the kernels.

The parameter names (``attn_norm_weight``, ``mlp_norm_weight``, ``qkv_proj``,
``out_proj``, ``mlp_up``, ``mlp_down``) and the QKV row order (q, then k,
then v) are the reference's, so state dicts load into either.
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
BACKEND_KERNELFORGE = "kernelforge"
BACKEND_KERNELO = BACKEND_KERNELFORGE  # earlier name, kept for existing callers
BACKENDS = (BACKEND_TORCH, BACKEND_KERNELFORGE)


@dataclass(frozen=True)
class BlockConfig:
    """Block geometry. Defaults are Llama-2-7B's matrix shapes (hidden 4096, 32
    heads, MLP 11008); the MLP is GELU rather than SwiGLU because the fused
    epilogue is bias + tanh-GELU."""

    hidden: int = 4096
    heads: int = 32
    intermediate: int = 11008
    eps: float = DEFAULT_EPS

    def __post_init__(self) -> None:
        if self.hidden % self.heads != 0:
            raise ValueError(f"hidden {self.hidden} is not divisible by {self.heads} heads")

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


class _TorchPath:
    """The swappable operators in plain PyTorch."""

    def norm(self, block: TransformerBlock, rows: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        return rmsnorm_reference(rows, weight, eps=block.config.eps)

    def up_gelu(self, block: TransformerBlock, rows: torch.Tensor) -> torch.Tensor:
        return F.gelu(block.mlp_up(rows), approximate="tanh")


class _KernelPath:
    """The swappable operators on this package's kernels, configured by dispatch.

    A configuration is looked up once per (operation, rows, dtype) and kept:
    dispatch reads cache files, and a block runs many forwards per shape.
    """

    def __init__(self, cache: ConfigCache | None) -> None:
        self.cache = cache
        self.chosen: dict[tuple[str, int, torch.dtype], KernelConfig] = {}

    def _config(self, block: TransformerBlock, operation: str, rows: int,
                dtype: torch.dtype) -> KernelConfig:
        key = (operation, rows, dtype)
        if key not in self.chosen:
            from kernelforge.kernels import get_operator

            geo = block.config
            if operation == "rmsnorm":
                problem = Problem.create(operation, dtype, rows=rows, cols=geo.hidden)
            else:  # the MLP weight is read as weight.t(): k-contiguous B
                problem = Problem.create(operation, dtype, layout="bt", M=rows,
                                         N=geo.intermediate, K=geo.hidden)
            self.chosen[key] = select_config(get_operator(operation), problem, cache=self.cache).config
        return self.chosen[key]

    def norm(self, block: TransformerBlock, rows: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        cfg = self._config(block, "rmsnorm", rows.shape[0], rows.dtype)
        return rmsnorm(rows, weight, eps=block.config.eps, config=cfg)

    def up_gelu(self, block: TransformerBlock, rows: torch.Tensor) -> torch.Tensor:
        cfg = self._config(block, "fused_linear", rows.shape[0], rows.dtype)
        # nn.Linear keeps its weight as (out, in); the transposed view is the
        # (K, N) operand with k-contiguous columns, read through its strides.
        return fused_linear_gelu(rows, block.mlp_up.weight.t(), block.mlp_up.bias, config=cfg)


class TransformerBlock(nn.Module):
    """Pre-norm decoder block: x + attn(norm(x)), then x + mlp(norm(x))."""

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
        self.config = config or BlockConfig()
        self._paths = {BACKEND_TORCH: _TorchPath(), BACKEND_KERNELFORGE: _KernelPath(cache)}
        self.backend = backend
        h, inter = self.config.hidden, self.config.intermediate
        opts = {"device": device, "dtype": dtype}
        self.attn_norm_weight = nn.Parameter(torch.ones(h, **opts))
        self.mlp_norm_weight = nn.Parameter(torch.ones(h, **opts))
        self.qkv_proj = nn.Linear(h, 3 * h, bias=False, **opts)
        self.out_proj = nn.Linear(h, h, bias=False, **opts)
        self.mlp_up = nn.Linear(h, inter, bias=True, **opts)
        self.mlp_down = nn.Linear(inter, h, bias=False, **opts)

    @property
    def backend(self) -> str:
        return self._backend

    @backend.setter
    def backend(self, value: str) -> None:
        if value not in BACKENDS:
            raise ValueError(f"backend must be one of {BACKENDS}, got {value!r}")
        self._backend = value

    def _attention(self, rows: torch.Tensor, batch: int, seq: int) -> torch.Tensor:
        geo = self.config
        # (tokens, 3*hidden) -> three (batch, heads, seq, head_dim) views.
        q, k, v = (self.qkv_proj(rows).view(batch, seq, 3, geo.heads, geo.head_dim)
                   .permute(2, 0, 3, 1, 4).unbind(0))
        mixed = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.out_proj(mixed.transpose(1, 2).reshape(batch * seq, geo.hidden))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() != 3:
            raise ValueError(f"expected (batch, seq, hidden), got {tuple(x.shape)}")
        batch, seq, width = x.shape
        if width != self.config.hidden:
            raise ValueError(f"expected hidden {self.config.hidden}, got {width}")
        path = self._paths[self._backend]
        rows = x.reshape(batch * seq, width)
        rows = rows + self._attention(path.norm(self, rows, self.attn_norm_weight), batch, seq)
        mlp = self.mlp_down(path.up_gelu(self, path.norm(self, rows, self.mlp_norm_weight)))
        return (rows + mlp).view(batch, seq, width)


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
    """The latency distribution of one block forward per backend, same weights and input.

    Unflushed: at the default geometry the block reads about 300 MiB of fp16
    weights per forward, more than L2 and the Infinity Cache hold, so every
    iteration already starts cold.
    """
    from kernelforge.benchmark.runner import benchmark

    block = TransformerBlock(config, dtype=dtype, device=device, cache=cache)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(batch, seq, block.config.hidden, generator=g).to(device=device, dtype=dtype)
    timings: dict[str, object] = {}
    with torch.inference_mode():
        for name in BACKENDS:
            block.backend = name
            timings[name] = benchmark(lambda: block(x), warmup=warmup, iterations=iterations,
                                      device=device, flush_l2=False)
    return timings
