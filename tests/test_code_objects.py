"""Compile-time properties of our own gfx950 code objects (no GPU needed).

The reference asserts on NVIDIA compiler output (tensor-core instructions, one
exp per epilogue element, shared-memory sizes, no local memory). The same
intent is checked here on the AMD code objects inside libkernelforge_hip.so:
kernel metadata from ``llvm-readelf --notes`` and instructions from
``llvm-objdump -d`` of code this repository compiled.
"""

from __future__ import annotations

import re

import pytest

from codeobj import load_kernels
from kernelforge.runtime import hip
from kernelforge.tuning.search import (
    REGISTER_FILE_PER_LANE,
    gemm_direct_static_lds_bytes,
    gemm_instantiations,
    mfma_fragment_edge,
)


@pytest.fixture(scope="module")
def kernels():
    hip.load()  # fails loudly if the library is not built
    return load_kernels(str(hip.LIBRARY_PATH))


def _gemm_params(name):
    m = re.search(r"gemm_(direct_)?kernelI(f|DF16_|DF16b)((?:Li\d+E)+)", name)
    if not m:
        return None
    ints = [int(x) for x in re.findall(r"Li(\d+)E", m.group(3))]
    dtype = {"f": "fp32", "DF16_": "fp16", "DF16b": "bf16"}[m.group(2)]
    return bool(m.group(1)), dtype, ints


def test_every_kernel_is_present(kernels):
    staged = gemm_instantiations()
    direct = gemm_instantiations(direct=1)
    n_gemm = 3 * (len(staged[4]) + 2 * len(staged[2])) + 2 * (len(direct[4]) + 2 * len(direct[2]))
    gemm = [n for n in kernels if _gemm_params(n)]
    assert len(gemm) == n_gemm
    assert sum("softmax_rows" in n for n in kernels) == 3 * 7
    assert sum("rmsnorm_rows" in n for n in kernels) == 3 * 7
    assert sum("gemv_splitk" in n for n in kernels) == 3 * 4 * 4  # dtypes x row counts x strip widths
    assert sum("gemv_dot" in n for n in kernels) == 3 * 4 * 4  # dtypes x row counts x lanes per column
    assert sum("rmsnorm_two_pass" in n for n in kernels) == 3 * 4 * 2  # dtypes x unrolls x staging
    assert sum("vector_add_kernel" in n for n in kernels) == 3 * 7  # dtypes x elements per lane


def test_no_kernel_spills_to_scratch(kernels):
    spilled = {n: k.private_bytes for n, k in kernels.items() if k.private_bytes}
    assert not spilled


def test_register_use_stays_in_the_file(kernels):
    for name, k in kernels.items():
        assert k.vgprs + k.agprs <= REGISTER_FILE_PER_LANE, name


def test_mfma_instructions_match_the_dtype_and_tile(kernels):
    expect = {"fp16": "v_mfma_f32_16x16x32_f16", "bf16": "v_mfma_f32_16x16x32_bf16",
              "fp32": "v_mfma_f32_16x16x4_f32"}
    wide = {"fp16": "v_mfma_f32_32x32x16_f16", "bf16": "v_mfma_f32_32x32x16_bf16"}
    seen_wide = 0
    for name, k in kernels.items():
        p = _gemm_params(name)
        if not p:
            continue
        direct, dtype, ints = p
        if direct and mfma_fragment_edge(ints[0], ints[1], direct=1) == 32:
            # 256x256: 64x128 wave tiles of 32x32x16 products, 4 k steps x 8 per slice
            assert k.count(wide[dtype]) > 0 and k.count(expect[dtype]) == 0, name
            seen_wide += 1
        else:
            assert k.count(expect[dtype]) > 0, name
    assert seen_wide == 2 * 2  # fp16, bf16 x both B layouts


def test_direct_kernels_use_dma_and_transposing_reads(kernels):
    seen = 0
    for name, k in kernels.items():
        p = _gemm_params(name)
        if not p or not p[0]:
            continue
        seen += 1
        direct, dtype, (bm, bn, waves, blayout, stages) = p
        assert k.count("global_load_lds_dwordx4") > 0, name
        if blayout == 0:
            # n-contiguous B: transposing reads for 16-bit elements; fp32 reads
            # a column's k-rows four bytes per lane and never transposes.
            if dtype == "fp32":
                reads = sum(k.count(op) for op in ("ds_read_b32", "ds_read2_b32", "ds_read2st64_b32"))
                assert reads > 0 and k.count("ds_read_b64_tr_b16") == 0, name
            else:
                assert k.count("ds_read_b64_tr_b16") > 0, name
        # Static LDS = the search space's model of the dense stages (or the
        # 256x256 tile's staged C), <= 160 KiB.
        assert k.group_bytes == gemm_direct_static_lds_bytes(bm, bn, stages) <= 160 * 1024, name
    assert seen > 0


def test_staged_kernels_use_dynamic_lds_only(kernels):
    for name, k in kernels.items():
        p = _gemm_params(name)
        if p and not p[0]:
            assert k.group_bytes == 0, name  # sized at launch from the tile model


def test_gelu_epilogue_is_one_exp_per_output_element(kernels):
    for name, k in kernels.items():
        p = _gemm_params(name)
        if not p or p[0] or p[1] != "fp16":
            continue
        bm, bn, bk, waves, _, _ = p[2]
        wm, wn = (2, 2) if waves == 4 else ((4, 2) if bm >= bn else (2, 4))
        per_lane = (bm // wm) * (bn // wn) // 64
        assert k.count("v_exp_f32") == per_lane, name


def test_softmax_is_one_exp_per_element(kernels):
    for name, k in kernels.items():
        m = re.search(r"softmax_rowsI\w+?Li(\d+)E", name)
        if m:
            assert k.count("v_exp_f32") == int(m.group(1)) * _row_copies(name), name


def _row_copies(name):
    """Row loops in the code object. Softmax rows of 1-4 vectors per lane carry a
    second, prefetching copy of the loop (rows.hip prefetch_rows); RMSNorm has a
    separate vector-path loop whenever a lane holds at least one whole vector
    (it issues gamma's loads behind the first row's)."""
    m = re.search(r"_rowsI(f|DF16_|DF16b)Li(\d+)E", name)
    size = 4 if m.group(1) == "f" else 2
    ept = int(m.group(2))
    if "rmsnorm_rows" in name:
        return 2 if ept * size >= 16 else 1
    return 2 if (ept >= 16 // size and ept * size <= 64) else 1


def test_row_reductions_use_cross_lane_ops_and_one_barrier_per_reduction(kernels):
    for name, k in kernels.items():
        if "softmax_rows" in name:
            assert k.count("s_barrier") == 2 * _row_copies(name), name  # max, then sum
        if "rmsnorm_rows" in name:
            assert k.count("s_barrier") == 1 * _row_copies(name), name
        if "_rows" in name:
            xlane = sum(k.count(op) for op in ("ds_bpermute_b32", "ds_swizzle_b32", "v_permlane32_swap_b32",
                                               "v_permlane16_swap_b32")) + sum(
                1 for line in k.asm if "row_" in line or "quad_perm" in line)
            assert xlane >= 6, name


def _operands(line):
    return line.split("//")[0]


def test_split_k_partials_move_with_the_agent_coherent_cache_policy(kernels):
    """Split-K partial sums cross XCDs, whose L2s are not coherent with each
    other. The protocol relies on every partial store and load carrying sc1
    (what the compiler emits for an agent-scope atomic store or load on gfx950),
    so a compiler that dropped it would show up here rather than as stale sums.

    * GEMV (16-bit, one x row): 32-bit global stores and loads touch only the
      workspace (y is 16-bit, x and W are read as vectors), so every one must
      carry sc1; the ticket is an atomic add that returns its value.
    * Direct GEMM: the partial tiles move through 16-byte buffer stores and
      loads, the only buffer accesses in the kernel.
    """
    seen_gemv = seen_gemm = 0
    for name, k in kernels.items():
        if re.search(r"gemv_(splitk|dot)IDF16[_b]Li1E", name):
            ops = [l for l in k.asm if l.split(None, 1)[0] in ("global_store_dword", "global_load_dword")]
            assert ops, name
            assert all("sc1" in _operands(l) for l in ops), (name, [l for l in ops if "sc1" not in l])
            atomics = [l for l in k.asm if l.split(None, 1)[0].startswith("global_atomic_add")]
            assert len(atomics) == 1 and "sc0" in _operands(atomics[0]), name
            seen_gemv += 1
        params = _gemm_params(name)
        if params and params[0]:
            ops = [l for l in k.asm if l.split(None, 1)[0] in ("buffer_store_dwordx4", "buffer_load_dwordx4")]
            assert ops, name
            assert all("sc1" in _operands(l) for l in ops), name
            seen_gemm += 1
    assert seen_gemv == 2 * 2 * 4 and seen_gemm > 0


def test_direct_gemm_writes_its_staged_c_tile_non_temporally(kernels):
    """The direct kernels store C's 16-byte row pieces with the non-temporal
    policy (written once, not read back by the launch); measured 0.5-3% faster
    than plain stores on the large shapes, with the same outputs. A tile whose
    staged C (BLOCK_M rows of BLOCK_N + 16 bytes) exceeds its LDS stages -- some
    fp32 tiles -- stores element by element and has no 16-byte row pieces."""
    seen = 0
    for name, k in kernels.items():
        p = _gemm_params(name)
        if not p or not p[0]:
            continue
        _, dtype, (bm, bn, waves, blayout, stages) = p
        elem = 4 if dtype == "fp32" else 2
        stores = [l for l in k.asm if l.split(None, 1)[0] == "global_store_dwordx4"]
        if bm * (bn + 16 // elem) * elem > gemm_direct_static_lds_bytes(bm, bn, stages):
            assert not any(" nt" in _operands(l) for l in stores), name
            continue
        assert any(" nt" in _operands(l) for l in stores), name
        seen += 1
    assert seen >= 2 * 2 * len(gemm_instantiations(direct=1)[2])
