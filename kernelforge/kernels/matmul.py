"""GEMM ``C = A @ B`` on gfx950 MFMA, plus the split-K GEMV for decode rows.

Python surface of the reference's ``matmul`` (kernelforge/kernels/matmul.py:
118-259): same signature, same validation messages (``_check_operands``,
:123-129), output allocated with ``torch.empty`` in the input dtype, any
operand strides accepted. The device work is one call into
``libkernelforge_hip.so``: ``kf_gemm`` (MFMA tiles), ``kf_gemm_split_k`` (the
same tiles with K shared out over ``SPLIT_K`` programs per tile, for row
counts whose tiles leave CUs idle) or, when the config carries ``GEMV=1``,
``kf_gemv`` (split-K, HBM-bound, M <= 8).
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
from kernelforge.testing import exact_fp32_matmul
from kernelforge.runtime.dispatch import shipped_config
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import GEMV_DEFAULT_LANES_PER_ROW, MatmulSearchSpace

#: A mid-size tile compiled for every dtype: the fixed, always-feasible
#: configuration (the reference's DEFAULT_CONFIG, matmul.py:118-120).
DEFAULT_CONFIG = KernelConfig(
    "matmul", BLOCK_M=128, BLOCK_N=128, BLOCK_K=64, GROUP_M=8, num_warps=4, num_stages=2
)


def _check_operands(a: torch.Tensor, b: torch.Tensor) -> None:
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError(f"expected 2D operands, got {tuple(a.shape)} and {tuple(b.shape)}")
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"shape mismatch for matmul: {tuple(a.shape)} @ {tuple(b.shape)}")
    if a.dtype != b.dtype:
        raise ValueError(f"dtype mismatch: {a.dtype} vs {b.dtype}")


def operand_layout(b: torch.Tensor) -> str:
    """``"bt"`` when B is read k-contiguous (an ``nn.Linear`` weight passed as
    ``weight.t()``), else ``""``: the problem layout whose winners apply."""
    return "bt" if b.stride(0) == 1 and b.shape[0] > 1 and b.stride(1) != 1 else ""


def default_gemm_config(operation: str, a: torch.Tensor, b: torch.Tensor) -> KernelConfig:
    """What an entry point runs without ``config=``: the shipped winner for
    the shape and B's layout, else the search space's heuristic. A product
    over k-contiguous B with no winner of its own borrows the row-major
    winner for MFMA tiles (their pipelines read both layouts at the same
    speed), but not for the decode GEMV, whose kernel differs by layout."""
    m, k = a.shape
    n = b.shape[1]
    layout = operand_layout(b)
    cfg = shipped_config(operation, a.dtype, a.device, layout=layout, M=m, N=n, K=k)
    if cfg is None and layout and m > MatmulSearchSpace.GEMV_MAX_M:
        cfg = shipped_config(operation, a.dtype, a.device, M=m, N=n, K=k)
    return cfg or _heuristic_config(operation, m, n, k, a.dtype, layout)


@lru_cache(maxsize=1024)
def _heuristic_config(operation: str, m: int, n: int, k: int, dtype: torch.dtype,
                      layout: str = "") -> KernelConfig:
    """The search space's top-priority candidate for the MI355X model.

    Deterministic and device-free, so it is the same on every host. An empty
    dimension is planned as 1: the launch itself returns at once when M or N
    is zero.
    """
    from kernelforge.tuning.search import search_space

    problem = Problem.create(operation, dtype, layout=layout, M=max(m, 1), N=max(n, 1), K=max(k, 1))
    best = search_space(operation).candidates(problem, MI355X_CAPS, max_candidates=1)
    return best[0] if best else DEFAULT_CONFIG


def launch_gemm(
    a: torch.Tensor,
    b: torch.Tensor,
    bias: torch.Tensor | None,
    out: torch.Tensor,
    cfg: KernelConfig,
) -> torch.Tensor:
    """Enqueue ``out = a @ b`` (or ``gelu(a @ b + bias)``) on the current stream."""
    hip.require_device_tensor(a, b, out, *(t for t in (bias,) if t is not None))
    lib = hip.load()
    m, k = a.shape
    n = b.shape[1]
    epilogue = hip.KF_EPILOGUE_BIAS_GELU if bias is not None else hip.KF_EPILOGUE_NONE
    stream = hip.stream_of(a)
    code = abi_code(a.dtype)
    bias_ptr = bias.data_ptr() if bias is not None else None
    if cfg.get("GEMV"):
        split = cfg["SPLIT_K"]
        need = lib.kf_gemv_workspace_bytes(m, n, split)
        ws = hip.workspaces.get(a.device, stream, need) if need else None
        rc = lib.kf_gemv(
            code, a.data_ptr(), b.data_ptr(), bias_ptr, out.data_ptr(),
            m, n, k, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
            out.stride(0), out.stride(1), epilogue, split, cfg["num_warps"],
            cfg.get("LANES_PER_ROW", GEMV_DEFAULT_LANES_PER_ROW),
            ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
            stream,
        )
        hip.check(rc, "gemv")
        return out
    split = cfg.get("SPLIT_K", 1)
    if split > 1:
        need = lib.kf_gemm_workspace_bytes(m, n, cfg["BLOCK_M"], cfg["BLOCK_N"], split)
        ws = hip.workspaces.get(a.device, stream, need) if need else None
        rc = lib.kf_gemm_split_k(
            code, a.data_ptr(), b.data_ptr(), bias_ptr, out.data_ptr(),
            m, n, k, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
            out.stride(0), out.stride(1), epilogue,
            cfg["BLOCK_M"], cfg["BLOCK_N"], cfg["BLOCK_K"], cfg["num_warps"],
            cfg.get("num_stages", 2), cfg.get("GROUP_M", 8), split,
            ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
            stream,
        )
        hip.check(rc, "gemm")
        return out
    rc = lib.kf_gemm(
        code, a.data_ptr(), b.data_ptr(), bias_ptr, out.data_ptr(),
        m, n, k, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
        out.stride(0), out.stride(1), epilogue,
        cfg["BLOCK_M"], cfg["BLOCK_N"], cfg["BLOCK_K"], cfg["num_warps"],
        cfg.get("num_stages", 2), cfg.get("GROUP_M", 8),
        hip.KF_PIPELINE_DIRECT if cfg.get("DIRECT") else hip.KF_PIPELINE_STAGED, stream,
    )
    hip.check(rc, "gemm")
    return out


def gemm_availability(cfg: KernelConfig, dtype: torch.dtype) -> str:
    """Why the library cannot run ``cfg`` (tile family, pipeline) in ``dtype``, or ``""``.

    GEMV configurations select a kernel by template arguments that every
    build contains; tile configurations are looked up in the variant table.
    """
    if cfg.get("GEMV"):
        return ""
    direct = bool(cfg.get("DIRECT"))
    found = hip.load().kf_gemm_has_variant(
        abi_code(dtype), cfg["BLOCK_M"], cfg["BLOCK_N"], cfg["BLOCK_K"], cfg["num_warps"],
        cfg.get("num_stages", 2),
        hip.KF_PIPELINE_DIRECT if direct else hip.KF_PIPELINE_STAGED)
    if found:
        return ""
    return (f"no ahead-of-time instantiation of {cfg['BLOCK_M']}x{cfg['BLOCK_N']}x"
            f"{cfg['BLOCK_K']} with {cfg['num_warps']} waves, {cfg.get('num_stages', 2)} stages on "
            f"the {'direct' if direct else 'staged'} pipeline for {dtype}")


def matmul(a: torch.Tensor, b: torch.Tensor, *, config: KernelConfig | None = None) -> torch.Tensor:
    _check_operands(a, b)
    m, n = a.shape[0], b.shape[1]
    cfg = config or default_gemm_config("matmul", a, b)
    c = torch.empty((m, n), device=a.device, dtype=a.dtype)
    return launch_gemm(a, b, None, c, cfg)


class MatmulOperator(Operator):
    name = "matmul"
    config_order = (
        "BLOCK_M", "BLOCK_N", "BLOCK_K", "GROUP_M", "DIRECT", "GEMV", "SPLIT_K", "LANES_PER_ROW",
        "num_warps",
        "num_stages",
    )

    def search_space(self) -> MatmulSearchSpace:
        return MatmulSearchSpace()

    def make_inputs(
        self, problem: Problem, device: torch.device, *, seed: int = 0
    ) -> tuple[torch.Tensor, ...]:
        gen = cpu_generator(seed)
        dims = problem.dims_dict
        a = torch.randn(dims["M"], dims["K"], dtype=problem.dtype, generator=gen)
        b = torch.randn(dims["K"], dims["N"], dtype=problem.dtype, generator=gen)
        if problem.layout == "bt":  # B read k-contiguous, as from an nn.Linear weight
            return a.to(device), b.t().contiguous().to(device).t()
        return a.to(device), b.to(device)

    def reference(self, *inputs: torch.Tensor) -> torch.Tensor:
        a, b = inputs
        with exact_fp32_matmul():
            return torch.matmul(a, b)

    def run(self, config: KernelConfig, *inputs: torch.Tensor) -> torch.Tensor:
        a, b = inputs
        return matmul(a, b, config=config)

    def default_config(self, problem: Problem) -> KernelConfig:
        d = problem.dims_dict
        return _heuristic_config("matmul", d["M"], d["N"], d["K"], problem.dtype, problem.layout)

    def availability(self, config: KernelConfig, problem: Problem) -> str:
        return gemm_availability(config, problem.dtype)

    def flops(self, problem: Problem) -> int:
        d = problem.dims_dict
        return metrics.matmul_flops(d["M"], d["N"], d["K"])

    def bytes_moved(self, problem: Problem) -> int:
        d = problem.dims_dict
        return metrics.matmul_bytes(d["M"], d["N"], d["K"], problem.itemsize)

    def baselines(
        self, problem: Problem, inputs: tuple[torch.Tensor, ...]
    ) -> dict[str, Callable[[], torch.Tensor]]:
        a, b = inputs
        return {
            "torch_eager": lambda: torch.matmul(a, b),
            "hip_default": lambda: matmul(a, b, config=DEFAULT_CONFIG),
        }
