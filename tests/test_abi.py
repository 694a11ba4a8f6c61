"""The C-ABI boundary, without a GPU.

* libkernelforge_hip.so loads and exports every function include/kernelforge_hip.h
  declares, and the ctypes binding (kernelforge.runtime.hip.SIGNATURES)
  covers exactly that set.
* Calls that never reach the HIP runtime behave as documented: version and
  target queries, the variant table (which must equal the search space's
  instantiation rules), workspace sizing, zero-size early returns and every
  argument error, each with its KF_ERR_* code and a kf_last_error() message.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from kernelforge.runtime import hip
from kernelforge.tuning.search import gemm_instantiations

HEADER = Path(__file__).resolve().parent.parent / "include" / "kernelforge_hip.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(kf_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    return hip.load()


def test_header_declares_the_expected_entry_points():
    assert _declared() == {
        "kf_abi_version", "kf_build_target", "kf_source_digest", "kf_last_error",
        "kf_stream_capture_id",
        "kf_gemm", "kf_gemm_has_variant", "kf_gemm_variant_count", "kf_gemm_variant_info",
        "kf_gemm_split_k", "kf_gemm_workspace_bytes", "kf_gemm_concurrent_tiles",
        "kf_gemv", "kf_gemv_workspace_bytes", "kf_gemv_no_alloc", "kf_softmax", "kf_rmsnorm",
        "kf_rmsnorm_two_pass", "kf_rmsnorm_two_pass_max_staged_cols", "kf_vector_add",
    }


def test_every_declared_symbol_is_exported_and_bound(lib):
    declared = _declared()
    assert declared == set(hip.SIGNATURES)
    for name in declared:
        assert getattr(lib, name) is not None  # AttributeError if not exported


def test_identification(lib):
    assert lib.kf_abi_version() == hip.ABI_VERSION == 5
    assert lib.kf_build_target() == b"gfx950"


def test_the_library_is_built_from_the_sources_in_the_tree(lib):
    """The digest the build compiled in is the digest of today's sources, tile
    lists and flags: a stale library (sources edited, not rebuilt) fails here,
    and profiles keyed on the digest can only describe this code."""
    from kernelforge import build

    digest = hip.source_digest()
    assert len(digest) == 16 and int(digest, 16) >= 0
    assert digest == build.source_digest()


def test_a_library_of_another_abi_version_is_refused(tmp_path):
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    src = tmp_path / "old.c"
    src.write_text("int kf_abi_version(void) { return 3; }\n")
    so = tmp_path / "libold.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    with pytest.raises(hip.KernelLibraryNotCompiled, match="ABI version 3"):
        hip.load(so)


def test_variant_table_equals_the_instantiation_rules(lib):
    staged = gemm_instantiations()
    direct = gemm_instantiations(direct=1)
    expected = set()
    for dt, elem in ((0, 4), (1, 2), (2, 2)):
        expected |= {(dt, *t, hip.KF_PIPELINE_STAGED) for t in staged[elem]}
        expected |= {(dt, *t, hip.KF_PIPELINE_DIRECT) for t in direct[elem]}
    got = hip.gemm_variants()
    assert len(got) == len(set(got)) == lib.kf_gemm_variant_count()
    assert set(got) == expected
    bm, bn, bk, w, s = staged[2][0]
    assert lib.kf_gemm_has_variant(1, bm, bn, bk, w, s, 0) == 1
    assert lib.kf_gemm_has_variant(1, 48, 48, 32, 4, 2, 0) == 0
    assert lib.kf_gemm_has_variant(0, 256, 128, 64, 8, 2, 1) == 0  # fp32 direct slices are 32 wide
    assert lib.kf_gemm_has_variant(0, 256, 128, 32, 8, 2, 1) == 1
    assert lib.kf_gemm_has_variant(0, 256, 256, 32, 8, 2, 1) == 0  # 32x32x16 is 16-bit only


def test_workspace_sizing(lib):
    assert lib.kf_gemv_workspace_bytes(1, 11008, 1) == 0
    # Every split-K workspace: a fixed 1 MiB counter region, then fp32 partials.
    counters = 1 << 20
    assert lib.kf_gemv_workspace_bytes(1, 11008, 8) == counters + 8 * 11008 * 4
    assert lib.kf_gemv_workspace_bytes(0, 11008, 8) == 0
    tiles = 1 * (11008 // 64)
    # Two partial tiles per split program, at most split_k programs per tile.
    assert lib.kf_gemm_workspace_bytes(32, 11008, 32, 64, 4) == counters + 2 * 4 * tiles * 32 * 64 * 4
    assert lib.kf_gemm_workspace_bytes(30, 11000, 32, 64, 4) == counters + 2 * 4 * tiles * 32 * 64 * 4
    assert lib.kf_gemm_workspace_bytes(32, 11008, 32, 64, 1) == 0
    assert lib.kf_gemm_workspace_bytes(0, 11008, 32, 64, 4) == 0


def _rc_and_message(rc_fn):
    rc = rc_fn()
    return rc, hip.last_error()


NULL = None


def test_gemm_argument_errors(lib):
    def gemm(dtype=1, m=64, n=64, k=64, epi=0, bm=64, bn=64, bk=64, w=4, st=2, gm=8, pipe=0,
             a=1 << 20, b=1 << 20, c=1 << 20, bias=NULL):
        return lib.kf_gemm(dtype, a, b, bias, c, m, n, k, k, 1, n, 1, n, 1, epi, bm, bn, bk, w, st,
                           gm, pipe, NULL)

    rc, msg = _rc_and_message(lambda: gemm(dtype=7))
    assert rc == hip.KF_ERR_UNSUPPORTED_DTYPE and "dtype" in msg
    rc, msg = _rc_and_message(lambda: gemm(m=-1))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "negative" in msg
    rc, msg = _rc_and_message(lambda: gemm(epi=9))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "epilogue" in msg
    rc, msg = _rc_and_message(lambda: gemm(gm=0))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "group_m" in msg
    rc, msg = _rc_and_message(lambda: gemm(pipe=5))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "pipeline" in msg
    rc, msg = _rc_and_message(lambda: gemm(bm=48))
    assert rc == hip.KF_ERR_NOT_BUILT and "no compiled" in msg
    rc, msg = _rc_and_message(lambda: gemm(epi=1))  # bias missing
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "bias" in msg
    # Zero-size problems return before any launch.
    assert gemm(m=0) == hip.KF_OK and gemm(n=0) == hip.KF_OK


def test_gemm_split_k_argument_errors(lib):
    def gemm(split=4, ws=NULL, wsb=0, m=64, n=64, k=256, dtype=1, bm=64, bn=64):
        return lib.kf_gemm_split_k(dtype, 1 << 20, 1 << 20, NULL, 1 << 20, m, n, k, k, 1, n, 1, n,
                                   1, 0, bm, bn, 64, 4, 3, 8, split, ws, wsb, NULL)

    need = lib.kf_gemm_workspace_bytes(64, 64, 64, 64, 4)
    rc, msg = _rc_and_message(lambda: gemm(split=0))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "split_k" in msg
    rc, msg = _rc_and_message(lambda: gemm(split=65))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "split_k" in msg
    rc, msg = _rc_and_message(lambda: gemm())
    assert rc == hip.KF_ERR_WORKSPACE and "workspace" in msg
    rc, msg = _rc_and_message(lambda: gemm(ws=1 << 20, wsb=need - 4))
    assert rc == hip.KF_ERR_WORKSPACE and str(need) in msg
    rc, msg = _rc_and_message(lambda: gemm(ws=(1 << 20) + 4, wsb=need))
    assert rc == hip.KF_ERR_WORKSPACE and "aligned" in msg
    # One counter per tile: more tiles than the counter region holds is refused.
    rc, msg = _rc_and_message(lambda: gemm(m=1 << 16, n=1 << 16, bm=64, bn=64))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "counters" in msg
    rc, msg = _rc_and_message(lambda: gemm(dtype=0))  # fp32 has no direct pipeline
    assert rc == hip.KF_ERR_NOT_BUILT and "direct" in msg
    # split_k is only meaningful on the direct pipeline: kf_gemm never splits,
    # and zero-size problems return before the workspace is looked at.
    assert gemm(m=0) == hip.KF_OK and gemm(n=0) == hip.KF_OK


def test_concurrent_tiles_query_errors(lib):
    rc = lib.kf_gemm_concurrent_tiles(7, 256, 128, 64, 8, 3, 1)
    assert rc == hip.KF_ERR_UNSUPPORTED_DTYPE
    rc, msg = _rc_and_message(lambda: lib.kf_gemm_concurrent_tiles(1, 48, 128, 64, 8, 3, 1))
    assert rc == hip.KF_ERR_NOT_BUILT and "no compiled" in msg


def test_gemv_argument_errors(lib):
    def gemv(m=1, n=64, k=64, split=1, waves=4, ws=NULL, wsb=0, dtype=2, epi=0, lanes=16):
        return lib.kf_gemv(dtype, 1 << 20, 1 << 20, NULL, 1 << 20, m, n, k, k, 1, n, 1, n, 1, epi,
                           split, waves, lanes, ws, wsb, NULL)

    rc, msg = _rc_and_message(lambda: gemv(m=9))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "decode limit" in msg
    rc, msg = _rc_and_message(lambda: gemv(waves=17))
    assert rc == hip.KF_ERR_OUT_OF_RESOURCES
    rc, msg = _rc_and_message(lambda: gemv(lanes=12))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "lanes_per_row" in msg
    rc, msg = _rc_and_message(lambda: gemv(split=0))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "split_k" in msg
    rc, msg = _rc_and_message(lambda: gemv(split=4))
    assert rc == hip.KF_ERR_WORKSPACE and "workspace" in msg
    rc, msg = _rc_and_message(lambda: gemv(split=4, n=(1 << 18) + 8))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "counters" in msg
    rc, msg = _rc_and_message(lambda: gemv(dtype=4))
    assert rc == hip.KF_ERR_UNSUPPORTED_DTYPE
    rc, msg = _rc_and_message(lambda: gemv(epi=1))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT
    assert gemv(m=0) == hip.KF_OK


def test_gemv_no_alloc_argument_errors(lib):
    """kf_gemv_no_alloc: kf_gemv's checks, plus the static scratch limit.

    Every case here returns before the library asks the runtime for anything
    (no device, no launch), so it runs without a GPU.
    """

    def gemv(m=1, n=64, k=64, split=1, waves=4, dtype=2, epi=0, lanes=16):
        return lib.kf_gemv_no_alloc(dtype, 1 << 20, 1 << 20, NULL, 1 << 20, m, n, k, k, 1, n, 1,
                                    n, 1, epi, split, waves, lanes, NULL)

    rc, msg = _rc_and_message(lambda: gemv(m=9, split=4))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "decode limit" in msg
    rc, msg = _rc_and_message(lambda: gemv(split=0))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "split_k" in msg
    rc, msg = _rc_and_message(lambda: gemv(lanes=12))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "lanes_per_row" in msg
    # The largest split the scratch holds, and one beyond it.
    limit = hip.KF_GEMV_NO_ALLOC_SCRATCH_BYTES - hip.KF_WORKSPACE_COUNTER_BYTES
    n = 11008
    fits = limit // (8 * n * 4)
    assert lib.kf_gemv_workspace_bytes(8, n, fits) <= hip.KF_GEMV_NO_ALLOC_SCRATCH_BYTES
    rc, msg = _rc_and_message(lambda: gemv(m=8, n=n, split=fits + 1))
    assert rc == hip.KF_ERR_WORKSPACE and "static scratch" in msg and str(hip.KF_GEMV_NO_ALLOC_SCRATCH_BYTES) in msg
    # Zero-size calls return without touching the scratch.
    assert gemv(m=0, split=4) == hip.KF_OK and gemv(n=0, split=4) == hip.KF_OK


def test_row_kernel_argument_errors(lib):
    def softmax(cols=100, block=128, rpp=1, waves=1, rows=4, dtype=1):
        return lib.kf_softmax(dtype, 1 << 20, 1 << 20, rows, cols, cols, cols, block, rpp, waves, NULL)

    rc, msg = _rc_and_message(lambda: softmax(block=64))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "cannot hold a row" in msg
    rc, msg = _rc_and_message(lambda: softmax(block=96))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "power of two" in msg
    rc, msg = _rc_and_message(lambda: softmax(cols=20000, block=32768, waves=16))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "single-pass limit" in msg
    rc, msg = _rc_and_message(lambda: softmax(waves=17))
    assert rc == hip.KF_ERR_OUT_OF_RESOURCES
    rc, msg = _rc_and_message(lambda: softmax(rpp=0))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT
    rc, msg = _rc_and_message(lambda: softmax(block=256, waves=3))
    assert rc == hip.KF_ERR_OUT_OF_RESOURCES and "per lane" in msg
    rc, msg = _rc_and_message(lambda: softmax(dtype=9))
    assert rc == hip.KF_ERR_UNSUPPORTED_DTYPE
    assert softmax(rows=0) == hip.KF_OK
    rc = lib.kf_rmsnorm(1, 1 << 20, 1 << 20, 1 << 20, 4, 100, 100, 100, ctypes.c_float(-1.0), 128,
                        1, 1, NULL)
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "eps" in hip.last_error()


def test_two_pass_rmsnorm_argument_errors(lib):
    def two_pass(cols=100_000, block=2048, rpp=1, waves=8, rows=4, dtype=0, stage=0, eps=1e-5):
        return lib.kf_rmsnorm_two_pass(dtype, 1 << 20, 1 << 20, 1 << 20, rows, cols, cols, cols,
                                       ctypes.c_float(eps), block, rpp, waves, stage, NULL)

    # fp32: 4 elements per 16-byte vector, so a trip is a multiple of waves*64*4.
    rc, msg = _rc_and_message(lambda: two_pass(block=1024))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "16-byte vectors per lane" in msg
    rc, msg = _rc_and_message(lambda: two_pass(block=3 * 2048))
    assert rc == hip.KF_ERR_NOT_BUILT and "vectors per lane per trip" in msg
    rc, msg = _rc_and_message(lambda: two_pass(waves=17, block=17 * 256))
    assert rc == hip.KF_ERR_OUT_OF_RESOURCES
    rc, msg = _rc_and_message(lambda: two_pass(waves=16, block=16 * 256 * 8))
    assert rc == hip.KF_ERR_OUT_OF_RESOURCES and "register pressure" in msg
    rc, msg = _rc_and_message(lambda: two_pass(stage=2))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "stage_row" in msg
    rc, msg = _rc_and_message(lambda: two_pass(eps=-1.0))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "eps" in msg
    rc, msg = _rc_and_message(lambda: two_pass(rpp=0))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT
    rc, msg = _rc_and_message(lambda: two_pass(dtype=5))
    assert rc == hip.KF_ERR_UNSUPPORTED_DTYPE
    # The staged row must fit the LDS a workgroup may hold.
    fp32_cols = lib.kf_rmsnorm_two_pass_max_staged_cols(0)
    assert fp32_cols == 159 * 1024 // 4
    assert lib.kf_rmsnorm_two_pass_max_staged_cols(1) == 2 * fp32_cols
    assert lib.kf_rmsnorm_two_pass_max_staged_cols(7) == 0
    rc, msg = _rc_and_message(lambda: two_pass(cols=fp32_cols + 4, stage=1))
    assert rc == hip.KF_ERR_OUT_OF_RESOURCES and "LDS" in msg
    assert two_pass(rows=0) == hip.KF_OK and two_pass(cols=0) == hip.KF_OK


def test_vector_add_argument_errors(lib):
    def vadd(n=1000, block=1024, waves=4, dtype=1):
        return lib.kf_vector_add(dtype, 1 << 20, 1 << 20, 1 << 20, n, block, waves, NULL)

    rc, msg = _rc_and_message(lambda: vadd(n=-1))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "negative" in msg
    rc, msg = _rc_and_message(lambda: vadd(block=100))
    assert rc == hip.KF_ERR_INVALID_ARGUMENT and "per lane" in msg
    rc, msg = _rc_and_message(lambda: vadd(block=768, waves=4))
    assert rc == hip.KF_ERR_NOT_BUILT and "elements per lane" in msg
    rc, msg = _rc_and_message(lambda: vadd(block=64 * 256, waves=2))
    assert rc == hip.KF_ERR_NOT_BUILT
    rc, msg = _rc_and_message(lambda: vadd(waves=0))
    assert rc == hip.KF_ERR_OUT_OF_RESOURCES
    rc, msg = _rc_and_message(lambda: vadd(dtype=3))
    assert rc == hip.KF_ERR_UNSUPPORTED_DTYPE
    assert vadd(n=0) == hip.KF_OK


def test_check_maps_codes_to_tuner_classified_exceptions():
    with pytest.raises(hip.KernelNotCompiled):
        hip.check(hip.KF_ERR_NOT_BUILT, "x")
    with pytest.raises(hip.KernelOutOfResources):
        hip.check(hip.KF_ERR_OUT_OF_RESOURCES, "x")
    with pytest.raises(hip.KernelOutOfMemoryError):
        hip.check(hip.KF_ERR_OUT_OF_MEMORY, "x")
    with pytest.raises(hip.KernelWorkspaceError):
        hip.check(hip.KF_ERR_WORKSPACE, "x")
    hip.check(hip.KF_OK, "x")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(hip.KernelLibraryNotCompiled, match="missing"):
        hip.load(tmp_path / "nope.so")
