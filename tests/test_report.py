"""Report generation from a seeded results database (no GPU needed).

The rows are fixtures chosen to reach every rendering path: two GEMM shapes
with tuned candidates over a tile plane, a memory-bound operator, two dtypes
at one shape, an incorrect fast row, mixed timing methods and an empty
database. Nothing here is a measurement. The behaviours checked are the
reference's (kernelforge/tests/test_report.py), with this build's labels.
"""

from __future__ import annotations

import pytest

from kernelforge.benchmark import report
from kernelforge.benchmark.runner import summarize
from kernelforge.db import Measurement, ResultsDB
from kernelforge.runtime.env import capture_environment
from kernelforge.testing import VerificationResult
from kernelforge.tuning.config import KernelConfig, Problem

pytest.importorskip("matplotlib")


def _timing(ms: float, *, flushed: bool = True, timer: str = "hip_event"):
    return summarize([ms * 0.97, ms, ms * 1.04], warmup=10, iterations=3, timer=timer,
                     flushed_l2=flushed)


def _ok():
    return VerificationResult(True, 1e-4, 1e-3, 0, 100, 5e-3)


def _tile(bm: int, bn: int) -> KernelConfig:
    return KernelConfig("matmul", BLOCK_M=bm, BLOCK_N=bn, BLOCK_K=64, GROUP_M=8, DIRECT=1,
                        num_warps=8, num_stages=2)


@pytest.fixture
def seeded(tmp_path):
    db = ResultsDB(tmp_path / "results.db")
    run = db.start_run(capture_environment(), notes="fixture", version="0.0.0")
    for (m, n, k), eager, mine in (((1024, 1024, 1024), 0.030, 0.024),
                                   ((2048, 4096, 4096), 0.075, 0.069)):
        problem = Problem.create("matmul", "fp16", M=m, N=n, K=k)
        flops = 2 * m * n * k
        for label, ms, cfg in (("torch_eager", eager, None), ("hip_default", mine * 1.3, _tile(128, 128)),
                               ("kernelforge", mine, _tile(128, 256))):
            db.record(run, problem, Measurement(label=label, status="ok", config=cfg,
                                                verification=_ok(), timing=_timing(ms),
                                                tflops=flops / (ms * 1e-3) / 1e12))
        for (bm, bn), factor in (((64, 64), 1.9), ((128, 128), 1.2), ((256, 128), 1.05)):
            ms = mine * factor
            db.record(run, problem, Measurement(label="kernelforge", status="ok", config=_tile(bm, bn),
                                                verification=_ok(), timing=_timing(ms),
                                                tflops=flops / (ms * 1e-3) / 1e12))
    rms = Problem.create("rmsnorm", "fp32", rows=4096, cols=4096)
    moved = (2 * 4096 * 4096 + 4096) * 4
    for label, ms in (("torch_eager", 0.061), ("kernelforge", 0.0266)):
        db.record(run, rms, Measurement(label=label, status="ok", verification=_ok(),
                                        timing=_timing(ms), gbps=moved / (ms * 1e-3) / 1e9))
    yield db
    db.close()


def test_summary_tables_and_figures_are_written(seeded, tmp_path):
    art = report.generate(seeded, tmp_path / "out")
    assert art.summary.exists()
    names = {p.name for p in art.figures}
    assert {"matmul_latency.png", "matmul_tflops.png", "rmsnorm_latency.png",
            "rmsnorm_bandwidth.png", "tuning_heatmap.png"} <= names
    assert "rmsnorm_tflops.png" not in names
    assert {p.name for p in art.tables} == {"matmul.csv", "rmsnorm.csv"}
    for p in art.figures:
        assert p.stat().st_size > 1000, p.name
    assert "summary.md" in art.render()


def test_rows_follow_problem_size_and_carry_speedup_and_peak_fraction(seeded, tmp_path):
    text = report.generate(seeded, tmp_path / "out").summary.read_text()
    assert text.index("| 1024x1024x1024 ") < text.index("| 2048x4096x4096 ")
    assert "## Environment" in text and "PyTorch" in text and "## matmul" in text
    assert "1.25x" in text  # 0.030 / 0.024
    # 2*2048*4096*4096 / 69 us = 995.9 TFLOP/s = 39.6% of 2516.6.
    assert "995.9" in text and "39.6%" in text
    # 134,234,112 B / 26.6 us = 5046.4 GB/s = 63.1% of 8000 GB/s.
    assert "GB/s" in text and "63.1%" in text


def test_fastest_row_per_label_is_reported(seeded, tmp_path):
    import csv

    report.generate(seeded, tmp_path / "out")
    with open(tmp_path / "out" / "matmul.csv") as fh:
        rows = list(csv.DictReader(fh))
    tuned = [r for r in rows if r["label"] == "kernelforge"]
    assert len(tuned) == 2  # one per shape, the fastest of four candidates
    assert sorted(round(float(r["median_us"]), 1) for r in tuned) == [24.0, 69.0]


def test_two_dtypes_at_one_shape_are_two_series(tmp_path):
    with ResultsDB(tmp_path / "r.db") as db:
        run = db.start_run(capture_environment())
        for dtype, ms in (("fp16", 1.0), ("bf16", 1.1)):
            p = Problem.create("matmul", dtype, M=512, N=512, K=512)
            for label, v in (("torch_eager", ms), ("kernelforge", ms * 0.8)):
                db.record(run, p, Measurement(label=label, status="ok", verification=_ok(),
                                              timing=_timing(v), tflops=1.0))
        art = report.generate(db, tmp_path / "out")
    text = art.summary.read_text()
    assert "fp16" in text and "bf16" in text
    assert next(p for p in art.figures if p.name == "matmul_latency.png").stat().st_size > 1000


def test_mixed_timing_methods_are_flagged(tmp_path):
    with ResultsDB(tmp_path / "r.db") as db:
        run = db.start_run(capture_environment())
        p = Problem.create("vector_add", "fp32", n=1 << 20)
        db.record(run, p, Measurement(label="torch_eager", status="ok", verification=_ok(),
                                      timing=_timing(0.01), gbps=1.0))
        db.record(run, p, Measurement(label="kernelforge", status="ok", verification=_ok(),
                                      timing=_timing(0.01, flushed=False), gbps=1.0))
        db.record(run, p, Measurement(label="torch_cpu", status="ok", verification=_ok(),
                                      timing=_timing(2.0, flushed=False, timer="perf_counter"),
                                      gbps=0.1))
        art = report.generate(db, tmp_path / "out")
    assert any("unflushed" in n for n in art.notes)
    assert any("only hip_event rows" in n for n in art.notes)
    text = art.summary.read_text()
    assert "Warning" in text and "PyTorch CPU" in text


def test_provenance_comes_from_the_latest_run(tmp_path):
    with ResultsDB(tmp_path / "r.db") as db:
        db.start_run(capture_environment(), notes="nothing recorded")
        art = report.generate(db, tmp_path / "out")
        assert "No runs recorded." not in art.summary.read_text()


def test_empty_database_says_so(tmp_path):
    with ResultsDB(tmp_path / "r.db") as db:
        art = report.generate(db, tmp_path / "out")
    assert "No correct, timed measurements" in art.summary.read_text()
    assert art.figures == [] and art.notes


def test_incorrect_rows_never_reach_a_table(tmp_path):
    with ResultsDB(tmp_path / "r.db") as db:
        run = db.start_run(capture_environment())
        p = Problem.create("matmul", "fp16", M=256, N=256, K=256)
        db.record(run, p, Measurement(
            label="kernelforge", status="incorrect",
            verification=VerificationResult(False, 1.0, 1.0, 50, 100, 5e-3, "wrong"),
            timing=_timing(0.0123)))
        db.record(run, p, Measurement(label="torch_eager", status="ok", verification=_ok(),
                                      timing=_timing(0.1)))
        text = report.generate(db, tmp_path / "out").summary.read_text()
    assert "PyTorch eager" in text and "12.3" not in text


def test_heatmap_is_skipped_without_tuned_gemm_candidates(tmp_path):
    with ResultsDB(tmp_path / "r.db") as db:
        run = db.start_run(capture_environment())
        p = Problem.create("rmsnorm", "fp16", rows=512, cols=512)
        db.record(run, p, Measurement(label="torch_eager", status="ok", verification=_ok(),
                                      timing=_timing(0.1)))
        art = report.generate(db, tmp_path / "out")
    assert any("tuning_heatmap" in n for n in art.notes)
    assert "tuning_heatmap.png" not in {p.name for p in art.figures}


def test_cli_report_renders_a_seeded_database(seeded, tmp_path):
    import subprocess
    import sys

    path = seeded.path
    out = subprocess.run(
        [sys.executable, "-m", "kernelforge", "report", "--db", str(path), "--out",
         str(tmp_path / "cli")],
        capture_output=True, text=True, timeout=300,
    )
    assert out.returncode == 0, out.stderr
    assert "measurements across" in out.stdout and (tmp_path / "cli" / "summary.md").exists()
