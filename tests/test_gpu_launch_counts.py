"""Device kernels per call, counted with the torch profiler on the GPU.

The structural claim behind the fused linear is a count, not a latency: the
unfused matmul + bias + GELU launches a GEMM, an add and an activation, the
fused kernel one (the reference asserts exactly this:
kernelforge/tests/test_fused_linear.py:176-204, through
kernelforge/profiling/pytorch_profiler.py:91-135).

The same count pins every entry point to a single launch per call at the
configurations bench.py times, and at the fused shape on a split-K tile. The
split-K GEMM and the split-K GEMV finish
their cross-program reduction inside that launch, and their counters are
reset by the kernel itself, so once a workspace exists no fill or memset
kernel runs ahead of a call.
"""

from __future__ import annotations

import pytest
import torch

from kernelforge.kernels import get_operator
from kernelforge.profiling import profile_kernels
from kernelforge.runtime.dispatch import SOURCE_PACKAGED, select_config
from kernelforge.tuning.config import Problem

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ours(name: str) -> bool:
    """True for a kernel of libkernelforge_hip.so (namespace kf), mangled or not."""
    return name.startswith("_ZN2kf") or "kf::" in name


def _packaged(operation: str, dtype: str, **dims):
    sel = select_config(get_operator(operation), Problem.create(operation, dtype, **dims),
                        device=DEV)
    assert sel.source == SOURCE_PACKAGED, f"{operation} {dims}: dispatch used {sel.source}"
    return sel.config


def _count(fn, label: str):
    res = profile_kernels(fn, label=label, warmup=5, iterations=10)
    print(res.render(), flush=True)
    return res


def test_fusion_reduces_the_kernel_launch_count():
    from kernelforge.kernels.fused_linear import (
        DEFAULT_CONFIG,
        fused_linear_gelu,
        linear_gelu_reference,
    )

    g = torch.Generator().manual_seed(0)
    x = torch.randn(1024, 1024, generator=g).to(torch.float16).to(DEV)
    w = (torch.randn(1024, 1024, generator=g) / 32).to(torch.float16).to(DEV)
    bias = torch.randn(1024, generator=g).to(torch.float16).to(DEV)
    unfused = _count(lambda: linear_gelu_reference(x, w, bias), "unfused")
    fused = _count(lambda: fused_linear_gelu(x, w, bias, config=DEFAULT_CONFIG), "fused")
    assert fused.launches_per_iteration == pytest.approx(1.0, abs=0.01)
    assert all(_ours(k.name) for k in fused.kernels), [k.name for k in fused.kernels]
    # A GEMM, a bias add and an activation at least; hipBLASLt may split its
    # GEMM further, which is its choice.
    assert unfused.launches_per_iteration >= 3.0


def _timed_cases():
    """(label, builder) for each configuration bench.py times; a builder
    returns the call to count, on the packaged winner that dispatch picks."""

    def gemm():
        from kernelforge.kernels.matmul import matmul

        cfg = _packaged("matmul", "fp16", M=2048, N=4096, K=4096)
        a = torch.randn(2048, 4096, device=DEV).div_(64).half()
        b = torch.randn(4096, 4096, device=DEV).div_(64).half()
        return lambda: matmul(a, b, config=cfg)

    def fused(split: bool):
        from kernelforge.kernels.fused_linear import fused_linear_gelu
        from kernelforge.tuning.config import KernelConfig

        if split:  # the 256x128 tile, last round split in two: the tail runs in this launch
            cfg = KernelConfig("fused_linear", BLOCK_M=256, BLOCK_N=128, BLOCK_K=64, DIRECT=1,
                               GROUP_M=4, SPLIT_K=2, num_stages=3, num_warps=8)
        else:
            cfg = _packaged("fused_linear", "fp16", M=4096, N=11008, K=4096)
        x = torch.randn(4096, 4096, device=DEV).div_(64).half()
        w = torch.randn(4096, 11008, device=DEV).div_(64).half()
        bias = torch.randn(11008, device=DEV).mul_(0.02).half()
        return lambda: fused_linear_gelu(x, w, bias, config=cfg)

    def gemv():
        from kernelforge.kernels.matmul import matmul

        cfg = _packaged("matmul", "bf16", M=1, N=11008, K=4096)
        assert cfg.get("SPLIT_K", 1) > 1, dict(cfg)
        x = torch.rand(1, 4096, device=DEV).mul_(2).sub_(1).bfloat16()
        w = torch.rand(4096, 11008, device=DEV).mul_(2).sub_(1).bfloat16()
        return lambda: matmul(x, w, config=cfg)

    def softmax():
        from kernelforge.kernels.softmax import softmax as run

        cfg = _packaged("softmax", "fp16", rows=8192, cols=4096)
        x = torch.randn(8192, 4096, device=DEV).mul_(3).half()
        return lambda: run(x, config=cfg)

    def rmsnorm():
        from kernelforge.kernels.rmsnorm import rmsnorm as run

        cfg = _packaged("rmsnorm", "fp32", rows=4096, cols=4096)
        x = torch.randn(4096, 4096, device=DEV)
        gamma = torch.randn(4096, device=DEV).mul_(0.1).add_(1)
        return lambda: run(x, gamma, eps=1e-6, config=cfg)

    def vector_add():
        from kernelforge.kernels.vector_add import vector_add as run

        cfg = _packaged("vector_add", "fp32", n=1 << 26)
        a = torch.randn(1 << 26, device=DEV)
        b = torch.randn(1 << 26, device=DEV)
        return lambda: run(a, b, config=cfg)

    return [("gemm_fp16_2048x4096x4096", gemm),
            ("fused_linear_fp16_4096x11008x4096", lambda: fused(False)),
            ("fused_linear_fp16_4096x11008x4096_split_k", lambda: fused(True)),
            ("gemv_bf16_1x11008x4096", gemv), ("softmax_fp16_8192x4096", softmax),
            ("rmsnorm_fp32_4096x4096", rmsnorm), ("vector_add_fp32_67108864", vector_add)]


@pytest.mark.parametrize("label,build", _timed_cases(), ids=[c[0] for c in _timed_cases()])
def test_one_launch_per_call_at_the_timed_configurations(label, build):
    print(f"launch count: {label}", flush=True)
    res = _count(build(), label)
    assert res.launches_per_iteration == pytest.approx(1.0, abs=0.01), res.render()
    assert all(_ours(k.name) for k in res.kernels), [k.name for k in res.kernels]
