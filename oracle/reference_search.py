"""Restatement of the reference's CUDA-era candidate rules -- TEST INFRASTRUCTURE ONLY.

Purpose: pin the *generic* candidate pipeline of kernelforge.tuning.search
(enumerate -> named rejections -> conditional utilisation prune -> priority
sort -> budget) against numbers the reference publishes. The reference's
GEMM space on A100 properties yields 432 grid points, 180 feasible, 180 after
the prune and 48 selected, with rejections 105 uncoalesced-A / 81
tile-too-small / 30 uncoalesced-B / 27 per-warp / 9 register pressure
(README.md:67-81); a 1x11008x4096 decode GEMM leaves 30 feasible
(README.md:91-94); RTX 4090 properties give 178 (README.md:95-96); and at
512x512x512 the prune removes 48 of 180 (README.md:229-230).

The rules below follow kernelforge/tuning/search.py:259-419 (grid :285-297,
shared-memory model :299-329, rules :340-394, priority :396-419) and are fed
through the product's own ``SearchSpace.generate``. They are not product
code: the product's gfx950 rules live in kernelforge/tuning/search.py.
"""

from __future__ import annotations

from collections.abc import Iterator
from itertools import product

from kernelforge.dtypes import itemsize
from kernelforge.runtime.env import DeviceCaps
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import SearchSpace, ceil_div

# search.py:49-67 (constants)
MAX_ACC_REGS_PER_THREAD = 128
MIN_ACC_REGS_PER_THREAD = 4
MIN_CONTIGUOUS_TILE_BYTES = 64


def a100_caps() -> DeviceCaps:
    """The reference's A100-80GB fixture (tests/conftest.py:29-45) as DeviceCaps."""
    return DeviceCaps(
        name="NVIDIA A100-SXM4-80GB",
        gcn_arch="sm80",
        total_memory_bytes=80 * 1024**3,
        cu_count=108,
        lds_per_workgroup=166912,
        lds_per_cu=167936,
        vgprs_per_lane=255,
        agprs_per_lane=0,
        max_threads_per_workgroup=1024,
        wave_size=32,
        xcd_count=1,
        l2_cache_bytes=40 * 1024 * 1024,
        mall_bytes=0,
        peak_fp16_tflops=312.0,
        peak_fp32_tflops=19.5,
        peak_hbm_gbps=2039.0,
    )


def rtx4090_caps() -> DeviceCaps:
    """The reference's RTX 4090 fixture (tests/conftest.py:48-64)."""
    return DeviceCaps(
        name="NVIDIA GeForce RTX 4090",
        gcn_arch="sm89",
        total_memory_bytes=24 * 1024**3,
        cu_count=128,
        lds_per_workgroup=101376,
        lds_per_cu=102400,
        vgprs_per_lane=255,
        agprs_per_lane=0,
        max_threads_per_workgroup=1024,
        wave_size=32,
        xcd_count=1,
        l2_cache_bytes=72 * 1024 * 1024,
        mall_bytes=0,
        peak_fp16_tflops=165.0,
        peak_fp32_tflops=82.6,
        peak_hbm_gbps=1008.0,
    )


class ReferenceGemmSpace(SearchSpace):
    """kernelforge/tuning/search.py:259-419 restated (Triton tiles, 32-lane warps)."""

    operation = "matmul"
    BLOCK_M = (16, 32, 64, 128)
    BLOCK_N = (16, 32, 64, 128)
    BLOCK_K = (16, 32, 64)
    NUM_WARPS = (2, 4, 8)
    NUM_STAGES = (2, 3, 4)
    GROUP_M = 8
    MIN_TILE_ELEMENTS = 1024

    def grid(self, problem: Problem) -> Iterator[KernelConfig]:
        for bm, bn, bk, warps, stages in product(
            self.BLOCK_M, self.BLOCK_N, self.BLOCK_K, self.NUM_WARPS, self.NUM_STAGES
        ):
            yield KernelConfig(
                self.operation,
                BLOCK_M=bm,
                BLOCK_N=bn,
                BLOCK_K=bk,
                GROUP_M=self.GROUP_M,
                num_warps=warps,
                num_stages=stages,
            )

    def num_programs(self, config: KernelConfig, problem: Problem) -> int:
        d = problem.dims_dict
        return ceil_div(d["M"], config["BLOCK_M"]) * ceil_div(d["N"], config["BLOCK_N"])

    def reject_reason(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> str | None:
        d = problem.dims_dict
        m, n, k = d["M"], d["N"], d["K"]
        bm, bn, bk = config["BLOCK_M"], config["BLOCK_N"], config["BLOCK_K"]
        width = itemsize(problem.dtype)
        smem = config["num_stages"] * bk * (bm + bn) * width
        if smem > caps.lds_per_workgroup:
            return f"shared memory: {smem // 1024} KiB exceeds the per-block limit"
        if bm * bn < self.MIN_TILE_ELEMENTS:
            return f"tile too small: {bm}x{bn} output elements per program"
        acc = bm * bn / (config["num_warps"] * 32)
        if acc > MAX_ACC_REGS_PER_THREAD:
            return f"register pressure: {acc:.0f} accumulator registers per thread"
        if acc < MIN_ACC_REGS_PER_THREAD:
            return f"too little work per thread: {acc:.1f} accumulator registers"
        if bm * bn < 256 * config["num_warps"]:
            return f"too little output per warp at num_warps={config['num_warps']}"
        if bk * width < MIN_CONTIGUOUS_TILE_BYTES:
            return f"uncoalesced A tile: BLOCK_K={bk} is {bk * width} contiguous bytes"
        if bn * width < MIN_CONTIGUOUS_TILE_BYTES:
            return f"uncoalesced B tile: BLOCK_N={bn} is {bn * width} contiguous bytes"
        if bm > 2 * m and bm > min(self.BLOCK_M):
            return f"tile overshoot: BLOCK_M={bm} for M={m}"
        if bn > 2 * n and bn > min(self.BLOCK_N):
            return f"tile overshoot: BLOCK_N={bn} for N={n}"
        k_iters = ceil_div(k, bk)
        if config["num_stages"] > 2 and k_iters < config["num_stages"]:
            return f"pipeline cannot fill: {k_iters} K iterations"
        return None

    def priority(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> tuple[float, ...]:
        d = problem.dims_dict
        bm, bn = config["BLOCK_M"], config["BLOCK_N"]
        programs = min(self.num_programs(config, problem), caps.cu_count)
        reuse = (bm * bn) / (bm + bn)
        padded = ceil_div(d["M"], bm) * bm * ceil_div(d["N"], bn) * bn
        return (-programs, -reuse, padded / (d["M"] * d["N"]))
