"""The path from profiler output to the kernel figures bench.py prints, on the CPU.

kernelforge.profiling.bench_profiles cuts a rocprofv3 trace of a ``bench.py
--marks`` run into workloads at the marker fills and summarises each
workload's kernel; bench.py uses a summary only if it describes the library
build (source digest) and the configuration of the current run. Synthetic
rocprofv3 CSVs (the layouts of tests/test_rocprof.py) stand in for a GPU run.
"""

from __future__ import annotations

import csv
import importlib.util
import json
import sys
from pathlib import Path

import pytest

from kernelforge.profiling import bench_profiles as bp
from test_rocprof import COUNTER_HEADER, FILL, TRACE_HEADER

REPO = Path(__file__).resolve().parent.parent
MARK = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<signed char>>(int)"
COPY = "__amd_rocclr_copyBuffer"
REDUCE = "void at::native::reduce_kernel<512, 1, at::native::ReduceOp<float, at::native::sum>>(int)"
GEMM = "_ZN2kf4gemm18gemm_direct_kernelIDF16_Li128ELi256ELi8ELi0ELi3EEEvNS0_4ArgsE"
GEMM_OTHER = "_ZN2kf4gemm18gemm_direct_kernelIDF16_Li256ELi128ELi8ELi0ELi3EEEvNS0_4ArgsE"
ROWS = "void kf::(anonymous namespace)::rmsnorm_rows<float, 16>(float const*, ...)"


def _bench():
    spec = importlib.util.spec_from_file_location("bench_module", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules.setdefault("bench_module", mod)
    spec.loader.exec_module(mod)
    return mod


# A bench run: marker, then the workload's launches (flushes, a torch comparator,
# the workload's kernel several times). (kernel, grid, duration ns)
RUN = [
    (MARK, 256, 1_000),
    (REDUCE, 4096, 80_000), (COPY, 131072, 400_000), (REDUCE, 4096, 80_000),
    (COPY, 131072, 398_000), (COPY, 131072, 402_000),
    (MARK, 512, 1_000),
    (ROWS, 1048576, 21_000), (REDUCE, 4096, 80_000), (ROWS, 1048576, 22_000),
    (ROWS, 1048576, 21_500), (FILL, 64, 2_000),
    (MARK, 768, 1_000),
    (GEMM_OTHER, 131072, 90_000),  # e.g. a gate launch of another tile: launched less often
    (GEMM, 131072, 61_000), (REDUCE, 4096, 80_000), (GEMM, 131072, 60_000),
    (GEMM, 131072, 62_000),
]
MARKS = {"library_digest": "0123456789abcdef", "workloads": [
    {"name": "hbm_copy_1GiB", "config": None, "kernel_hint": "copy", "copy_bytes": 1 << 30,
     "algorithmic_bytes": 2 << 30},
    {"name": "rmsnorm_fp32_4096x4096", "config": {"BLOCK_SIZE": 4096, "num_warps": 4},
     "algorithmic_bytes": 134234112},
    {"name": "gemm_fp16_2048x4096x4096", "config": {"BLOCK_M": 128, "BLOCK_N": 256},
     "algorithmic_bytes": 67108864},
]}


def _trace(path, run=RUN):
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(TRACE_HEADER)
        t = 1_000_000
        for i, (kernel, grid, ns) in enumerate(run, start=1):
            w.writerow(["KERNEL_DISPATCH", "Agent 1", 1, 0, 7, i, 3, kernel, i, t, t + ns, 0, 0,
                        64, 0, 40, 256, 1, 1, grid, 1, 1])
            t += ns + 5_000
    return path


def _counters(path, counter, values):
    """One counter per dispatch of RUN: values[kernel] (KiB)."""
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(COUNTER_HEADER)
        for i, (kernel, grid, _) in enumerate(RUN, start=1):
            w.writerow([i, i, "Agent 1", 1, 7, 7, grid, 3, kernel, 256, 0, 0, 64, 0, 40, counter,
                        f"{values.get(kernel, 1.0):.6f}", 1000, 2000])
    return path


def test_markers_cut_the_run_and_each_workload_takes_its_most_launched_kernel(tmp_path):
    out = bp.summarize_trace(MARKS, _trace(tmp_path / "t_kernel_trace.csv"))
    assert list(out) == ["hbm_copy_1GiB", "rmsnorm_fp32_4096x4096", "gemm_fp16_2048x4096x4096"]
    copy = out["hbm_copy_1GiB"]
    assert copy["kernel"] == COPY and copy["dispatches"] == 3 and copy["median_us"] == 400.0
    rows = out["rmsnorm_fp32_4096x4096"]
    assert rows["kernel"] == ROWS and rows["dispatches"] == 3 and rows["median_us"] == 21.5
    gemm = out["gemm_fp16_2048x4096x4096"]
    assert gemm["kernel"] == GEMM and gemm["grid"] == 131072 and gemm["dispatches"] == 3
    assert gemm["median_us"] == 61.0 and gemm["min_us"] == 60.0
    assert gemm["config"] == {"BLOCK_M": 128, "BLOCK_N": 256}
    assert bp.is_marker(MARK) and not bp.is_marker(FILL)
    assert not bp.is_marker(MARK.replace("signed char", "unsigned char"))  # torch's uint8 fills


def test_a_marks_file_from_another_run_is_refused(tmp_path):
    marks = {**MARKS, "workloads": MARKS["workloads"][:2]}
    with pytest.raises(ValueError, match="3 marker dispatches for 2 workloads"):
        bp.summarize_trace(marks, _trace(tmp_path / "t_kernel_trace.csv"))


def test_traffic_is_scaled_by_the_copy_calibration(tmp_path):
    # The copy reads 1 GiB and writes 1 GiB; its counters read 512 MiB and 1024 MiB.
    fetch = _counters(tmp_path / "f.csv", "FETCH_SIZE", {COPY: 512 * 1024, ROWS: 32 * 1024,
                                                          GEMM: 72 * 1024})
    write = _counters(tmp_path / "w.csv", "WRITE_SIZE", {COPY: 1024 * 1024, ROWS: 64 * 1024,
                                                          GEMM: 16 * 1024})
    doc = bp.summarize_traffic(MARKS, fetch, write)
    cal = doc["calibration"]
    assert cal["fetch_scale"] == pytest.approx(2.0) and cal["write_scale"] == pytest.approx(1.0)
    gemm = doc["kernels"]["gemm_fp16_2048x4096x4096"]
    assert gemm["fetch_bytes"] == pytest.approx(144 * 2**20)
    assert gemm["traffic_bytes"] == pytest.approx(160 * 2**20)
    assert gemm["kernel"] == GEMM


def test_the_summariser_writes_what_bench_reads(tmp_path):
    marks = tmp_path / "marks.json"
    marks.write_text(json.dumps(MARKS))
    trace = _trace(tmp_path / "t_kernel_trace.csv")
    fetch = _counters(tmp_path / "f.csv", "FETCH_SIZE", {COPY: 512 * 1024})
    write = _counters(tmp_path / "w.csv", "WRITE_SIZE", {COPY: 1024 * 1024})
    out = tmp_path / "profiles"
    assert bp.main(["--marks", str(marks), "--trace", str(trace), "--fetch", str(fetch),
                    "--write", str(write), "--trace-command", "rocprofv3 --kernel-trace ...",
                    "--out", str(out)]) == 0
    for name in ("kernel_trace.json", "hbm_traffic.json", "bench_workloads_kernel_trace.md",
                 "hbm_traffic_bench_workloads.md"):
        assert (out / name).exists(), name
    bench = _bench()
    cfg = {"BLOCK_M": 128, "BLOCK_N": 256}
    entry, why = bench.profile_entry(out / "kernel_trace.json", "gemm_fp16_2048x4096x4096", cfg,
                                     MARKS["library_digest"])
    assert why is None and entry["median_us"] == 61.0
    md = (out / "bench_workloads_kernel_trace.md").read_text()
    assert "rocprofv3 --kernel-trace ..." in md and "kernelforge.profiling.bench_profiles" in md


def test_bench_nulls_a_profile_of_another_configuration_or_build(tmp_path):
    """A packaged winner that changed since the profile (or a rebuilt library)
    makes the profiled kernel figures stale: bench reports null and why."""
    bench = _bench()
    path = tmp_path / "kernel_trace.json"
    path.write_text(json.dumps({"library_digest": "aaaa", "kernels": {
        "gemm": {"kernel": GEMM, "grid": 131072, "median_us": 60.0, "config": {"BLOCK_M": 128}}}}))
    assert bench.profile_entry(path, "gemm", {"BLOCK_M": 128}, "aaaa")[1] is None
    entry, why = bench.profile_entry(path, "gemm", {"BLOCK_M": 256}, "aaaa")
    assert entry is None and "dispatch picked" in why
    entry, why = bench.profile_entry(path, "gemm", {"BLOCK_M": 128}, "bbbb")
    assert entry is None and "library sources aaaa" in why
    assert bench.profile_entry(path, "softmax", None, "aaaa")[0] is None
    assert "missing" in bench.profile_entry(tmp_path / "nope.json", "gemm", None, "aaaa")[1]


def test_committed_profiles_describe_the_packaged_configuration_and_this_build():
    """The committed summaries were made from this tree's library and the
    configurations dispatch picks today; changing a packaged winner nulls the
    entry (checked on a copy of the packaged table)."""
    from kernelforge import build
    from kernelforge.runtime.dispatch import packaged_cache
    from kernelforge.runtime.env import MI355X_CAPS
    from kernelforge.tuning.config import Problem

    bench = _bench()
    path = REPO / "profiles" / "kernel_trace.json"
    doc = json.loads(path.read_text())
    digest = build.source_digest()
    assert doc["library_digest"] == digest
    problem = Problem.create("matmul", "fp16", M=2048, N=4096, K=4096)
    # What dispatch picks on an MI355X: the packaged winner for the device's key.
    picked = dict(packaged_cache().get(problem, MI355X_CAPS.key))
    entry, why = bench.profile_entry(path, "gemm_fp16_2048x4096x4096", picked, digest)
    assert why is None, why
    changed = {**picked, "BLOCK_N": 128 if picked["BLOCK_N"] != 128 else 256}
    entry, why = bench.profile_entry(path, "gemm_fp16_2048x4096x4096", changed, digest)
    assert entry is None and "dispatch picked" in why


def test_counter_passes_give_per_workload_medians_and_the_derived_clock(tmp_path):
    """Any other counter pass (MFMA busy, LDS) is summarised the same way; with the
    kernel-trace durations beside it the table derives the shader clock and the
    matrix cores' share of busy cycles (2048x4096x4096 recorded on MI355X:
    29,284,538 busy CU cycles in 66.5 us = 1.72 GHz, 67,108,864 MFMA busy cycles
    = 57.3%)."""
    pmc = _counters(tmp_path / "busy.csv", "SQ_BUSY_CU_CYCLES", {GEMM: 29_284_538.0})
    rows = list(csv.reader(open(pmc)))
    with open(pmc, "a", newline="") as fh:  # a second counter of the same pass
        w = csv.writer(fh)
        for r in rows[1:]:
            w.writerow(r[:15] + ["SQ_VALU_MFMA_BUSY_CYCLES",
                                 "67108864.0" if r[8] == GEMM else "0.0"] + r[17:])
    got = bp.summarize_counters(MARKS, pmc)
    gemm = got["gemm_fp16_2048x4096x4096"]
    assert gemm["counters"] == {"SQ_BUSY_CU_CYCLES": 29_284_538.0, "SQ_VALU_MFMA_BUSY_CYCLES": 67_108_864.0}
    doc = {"commands": ["rocprofv3 --pmc ..."], "library_digest": "x", "kernels": got}
    md = bp.counters_markdown(doc, {"gemm_fp16_2048x4096x4096": 66.5})
    line = next(l for l in md.splitlines() if l.startswith("| gemm_fp16"))
    assert "1.72" in line and "57.3%" in line


def test_the_stats_table_names_each_workloads_kernel(tmp_path):
    """rocprofv3 --stats rows (one per kernel name over the whole run) come out
    by total time, with the workload whose kernel each one is."""
    stats = tmp_path / "bench_kernel_stats.csv"
    with open(stats, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"])
        w.writerow([REDUCE, 950, 81_664_163, 85962.3, 27.3, 78_550, 100_827, 5458.3])
        w.writerow([GEMM, 121, 7_388_284, 61060.2, 2.47, 59_712, 66_071, 1269.2])
        w.writerow([ROWS, 61, 1_320_000, 21639.3, 0.44, 20_100, 23_000, 500.0])
    traced = bp.summarize_trace(MARKS, _trace(tmp_path / "t_kernel_trace.csv"))
    rows = bp.summarize_stats(stats, traced, top=1)  # the top kernel, then the workloads' kernels
    assert [r["kernel"] for r in rows] == [REDUCE, GEMM, ROWS]
    assert rows[2]["workloads"] == ["rmsnorm_fp32_4096x4096"]
    assert rows[1]["workloads"] == ["gemm_fp16_2048x4096x4096"] and rows[0]["workloads"] == []
    assert rows[1]["average_us"] == pytest.approx(61.0602) and rows[1]["calls"] == 121
    md = bp.stats_markdown(rows, ["rocprofv3 --kernel-trace --stats ..."], "abc")
    assert "| gemm_fp16_2048x4096x4096 | 121 | 61.1 |" in md and "rocprofv3 --kernel-trace --stats" in md
