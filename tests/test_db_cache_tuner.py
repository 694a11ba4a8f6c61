"""Persistence (SQLite results, JSON winner cache), dispatch and the tuner.

The tuner is driven end to end on the CPU with a fake operator, as the
reference's tests/test_tuner.py does (:39-244): one mode per failure kind
(correct and fast, raises a compile-named error, raises a runtime error,
returns a wrong answer, correct but slow) and the checks that matter -- wrong
configs are never ranked, failures carry no timing, statuses are classified,
the budget is honoured, the DB and the cache are written.
"""

from __future__ import annotations

import json
import time
from collections.abc import Iterator

import pytest
import torch

from kernelforge.db import SCHEMA_VERSION, Measurement, ResultsDB
from kernelforge.kernels.base import Operator
from kernelforge.runtime.dispatch import select_config
from kernelforge.runtime.env import MI355X_CAPS, capture_environment
from kernelforge.tuning.cache import CACHE_VERSION, ConfigCache
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import SearchSpace
from kernelforge.tuning.tuner import (
    STATUS_COMPILE_ERROR,
    STATUS_INCORRECT,
    STATUS_OK,
    STATUS_OOM,
    STATUS_RUNTIME_ERROR,
    Tuner,
    _classify,
)


def _problem():
    return Problem.create("fake", "fp32", n=4096)


# --- results DB -----------------------------------------------------------------------


def test_db_round_trip_and_dedup(tmp_path):
    db = ResultsDB(tmp_path / "r.db")
    env = capture_environment()
    run = db.start_run(env, notes="t", version="x")
    cfg = KernelConfig("fake", MODE=0)
    db.record_many(run, _problem(), [
        Measurement(label="kernelforge", status=STATUS_OK, config=cfg, tflops=1.0),
        Measurement(label="kernelforge", status=STATUS_INCORRECT, config=cfg, error="bad"),
        Measurement(label="torch_eager", status=STATUS_OK),
    ])
    counts = db.counts()
    assert counts == {"runs": 1, "problems": 1, "configs": 1, "results": 3}
    rows = db.rows(operation="fake")
    assert [r["label"] for r in rows] == ["kernelforge", "kernelforge", "torch_eager"]
    assert rows[0]["digest"] == cfg.digest and rows[2]["params_json"] is None
    assert db.operations() == ["fake"]
    assert len(db.runs()) == 1
    db.close()


def test_db_schema_version_is_checked(tmp_path):
    path = tmp_path / "r.db"
    ResultsDB(path).close()
    import sqlite3

    con = sqlite3.connect(path)
    con.execute(f"PRAGMA user_version = {SCHEMA_VERSION + 1}")
    con.commit()
    con.close()
    with pytest.raises(RuntimeError, match="schema version"):
        ResultsDB(path)


#: The reference's table layout (kernelforge/db.py:35-99 there): the column
#: names and types a database it creates has. A file-format fixture, written
#: out here so this test can build such a file without the reference.
_REFERENCE_TABLES = {
    "runs": "run_id INTEGER PRIMARY KEY AUTOINCREMENT, timestamp TEXT NOT NULL, hostname TEXT, "
            "platform TEXT, python_version TEXT, torch_version TEXT, triton_version TEXT, "
            "cuda_version TEXT, driver_version TEXT, gpu_name TEXT, gpu_arch TEXT, "
            "gpu_memory_bytes INTEGER, sm_count INTEGER, device_key TEXT NOT NULL, "
            "kernelforge_version TEXT, notes TEXT NOT NULL DEFAULT ''",
    "problems": "problem_id INTEGER PRIMARY KEY AUTOINCREMENT, operation TEXT NOT NULL, "
                "shape_key TEXT NOT NULL, dtype TEXT NOT NULL, dims_json TEXT NOT NULL, "
                "UNIQUE (operation, shape_key, dtype)",
    "configs": "config_id INTEGER PRIMARY KEY AUTOINCREMENT, operation TEXT NOT NULL, "
               "digest TEXT NOT NULL, params_json TEXT NOT NULL, UNIQUE (operation, digest)",
    "results": "result_id INTEGER PRIMARY KEY AUTOINCREMENT, run_id INTEGER NOT NULL, "
               "problem_id INTEGER NOT NULL, config_id INTEGER, label TEXT NOT NULL, "
               "status TEXT NOT NULL, correct INTEGER, rel_error REAL, median_us REAL, "
               "mean_us REAL, std_us REAL, min_us REAL, max_us REAL, p95_us REAL, p99_us REAL, "
               "warmup INTEGER, iterations INTEGER, timer TEXT, flushed_l2 INTEGER, tflops REAL, "
               "gbps REAL, error TEXT NOT NULL DEFAULT ''",
}

#: How the reference records a run and reads results back (its column lists).
_REFERENCE_RUN_INSERT = (
    "INSERT INTO runs (timestamp, hostname, platform, python_version, torch_version, "
    "triton_version, cuda_version, driver_version, gpu_name, gpu_arch, gpu_memory_bytes, "
    "sm_count, device_key, kernelforge_version, notes) VALUES "
    "('t', 'h', 'p', '3.10', '2.4', '3.0', '12.4', '550', 'A100', 'sm_80', 1, 108, "
    "'NVIDIA_A100', '0.1', '')")
_REFERENCE_ROWS_SELECT = (
    "SELECT r.label, r.median_us, p.operation, c.digest, run.gpu_name, run.torch_version, "
    "run.triton_version, run.cuda_version, run.driver_version, run.sm_count, "
    "run.kernelforge_version FROM results AS r JOIN problems AS p ON p.problem_id = r.problem_id "
    "JOIN runs AS run ON run.run_id = r.run_id LEFT JOIN configs AS c ON c.config_id = r.config_id")


def test_db_opens_and_writes_a_file_the_reference_created(tmp_path):
    """A database created with the reference's tables is widened (two nullable
    columns) and recorded into; the reference's own statements keep working on
    it and on a file this build created."""
    import sqlite3

    path = tmp_path / "reference.db"
    con = sqlite3.connect(path)
    for table, body in _REFERENCE_TABLES.items():
        con.execute(f"CREATE TABLE {table} ({body})")
    con.execute("PRAGMA user_version = 1")
    con.execute(_REFERENCE_RUN_INSERT)
    con.commit()
    con.close()

    env = capture_environment()
    with ResultsDB(path) as db:
        run = db.start_run(env, notes="mi355x", version="0.2")
        db.record_many(run, _problem(), [
            Measurement(label="kernelforge", status=STATUS_OK, config=KernelConfig("fake", MODE=0),
                        tflops=1.0)])
        (row,) = db.rows(operation="fake")
        assert row["label"] == "kernelforge" and row["triton_version"] is None
        assert [r["run_id"] for r in db.runs()] == [1, run]

    con = sqlite3.connect(path)
    ours = con.execute("SELECT sm_count, cu_count, hip_version, kernelforge_version, cuda_version "
                       "FROM runs WHERE run_id = ?", (run,)).fetchone()
    assert ours == (env.cu_count, env.cu_count, env.hip_version, "0.2", None)
    con.execute(_REFERENCE_RUN_INSERT)  # the reference writing into the widened table
    (read,) = con.execute(_REFERENCE_ROWS_SELECT).fetchall()
    assert read[0] == "kernelforge" and read[-2] == env.cu_count
    con.close()

    fresh = tmp_path / "ours.db"
    with ResultsDB(fresh) as db:
        db.record_many(db.start_run(env), _problem(), [Measurement("torch_eager", STATUS_OK)])
    con = sqlite3.connect(fresh)
    con.execute(_REFERENCE_RUN_INSERT)
    assert [r[0] for r in con.execute(_REFERENCE_ROWS_SELECT)] == ["torch_eager"]
    con.close()


def test_best_per_label_ignores_incorrect_rows(tmp_path):
    from kernelforge.benchmark.runner import summarize
    from kernelforge.testing import verify

    db = ResultsDB(":memory:")
    run = db.start_run(capture_environment())
    good = verify(torch.ones(2), torch.ones(2))
    bad = verify(torch.ones(2), torch.zeros(2))
    t = lambda ms: summarize([ms], warmup=0, iterations=1, timer="perf_counter", flushed_l2=False)
    db.record_many(run, _problem(), [
        Measurement("kernelforge", STATUS_OK, KernelConfig("fake", MODE=0), good, t(2.0)),
        Measurement("kernelforge", STATUS_INCORRECT, KernelConfig("fake", MODE=1), bad, t(1.0)),
    ])
    (best,) = db.best_per_label()
    assert best["median_us"] == pytest.approx(2000.0)


# --- winner cache ---------------------------------------------------------------------


def test_cache_round_trip_and_keys(tmp_path):
    path = tmp_path / "c.json"
    cache = ConfigCache(path)
    p16 = Problem.create("matmul", "fp16", M=1, N=2, K=3)
    pbf = Problem.create("matmul", "bf16", M=1, N=2, K=3)
    cfg = KernelConfig("matmul", BLOCK_M=32)
    cache.put(p16, "dev_a", cfg, median_us=1.5, timestamp="now", candidates_tested=7)
    again = ConfigCache(path)
    assert again.get(p16, "dev_a") == cfg
    assert again.get(p16, "dev_b") is None  # other hardware misses
    assert again.get(pbf, "dev_a") is None  # other dtype misses
    (entry,) = again.entries()
    assert entry.median_us == 1.5 and entry.candidates_tested == 7 and "dev_a" in entry.describe()
    assert json.loads(path.read_text())["version"] == CACHE_VERSION
    assert again.clear() == 1 and not path.exists() and len(again) == 0


def test_cache_refuses_corrupt_and_foreign_versions(tmp_path):
    bad = tmp_path / "bad.json"
    bad.write_text("{nope")
    with pytest.raises(RuntimeError, match="not valid JSON"):
        ConfigCache(bad)
    old = tmp_path / "old.json"
    old.write_text(json.dumps({"version": 99, "entries": {}}))
    with pytest.raises(RuntimeError, match="version 99"):
        ConfigCache(old)


def test_cache_write_is_atomic(tmp_path):
    path = tmp_path / "c.json"
    cache = ConfigCache(path)
    cache.put(Problem.create("matmul", "fp16", M=1, N=1, K=1), "d", KernelConfig("matmul", A=1))
    assert not list(tmp_path.glob("*.tmp"))


def test_packaged_winners_file_is_valid_and_keyed_for_mi355x():
    from kernelforge.tuning.cache import PACKAGED_CACHE

    cache = ConfigCache(PACKAGED_CACHE)
    keys = {e.device_key for e in cache.entries()}
    assert keys == {MI355X_CAPS.key}
    ops = {e.operation for e in cache.entries()}
    assert {"matmul", "fused_linear", "rmsnorm", "softmax"} <= ops


def test_dispatch_hit_packaged_and_default(tmp_path):
    from kernelforge.kernels import get_operator

    op = get_operator("matmul")
    problem = Problem.create("matmul", "fp16", M=64, N=64, K=64)
    cache = ConfigCache(tmp_path / "c.json")
    sel = select_config(op, problem, cache=cache)  # no GPU here: device key "cpu"
    assert sel.source == "default" and not sel.tuned and "default" in sel.describe()
    cfg = KernelConfig("matmul", BLOCK_M=32, BLOCK_N=32, BLOCK_K=32, num_warps=4, num_stages=2)
    cache.put(problem, sel.device_key, cfg)
    hit = select_config(op, problem, cache=cache)
    assert hit.tuned and hit.config == cfg


# --- the tuner, on a fake CPU operator ---------------------------------------------------

MODE_FAST, MODE_COMPILE, MODE_RUNTIME, MODE_WRONG, MODE_SLOW, MODE_OOM = range(6)


class KernelNotCompiled(RuntimeError):
    pass


class FakeOutOfMemoryError(RuntimeError):
    pass


class _FakeSpace(SearchSpace):
    operation = "fake"

    def grid(self, problem: Problem) -> Iterator[KernelConfig]:
        for mode in range(6):
            yield KernelConfig("fake", MODE=mode)
        yield KernelConfig("fake", MODE=99)  # rejected by rule

    def reject_reason(self, config, problem, caps):
        return "infeasible: mode 99" if config["MODE"] == 99 else None


class _FakeOperator(Operator):
    name = "fake"

    def search_space(self):
        return _FakeSpace()

    def make_inputs(self, problem, device, *, seed=0):
        g = torch.Generator().manual_seed(seed)
        return (torch.randn(problem["n"], generator=g),)

    def reference(self, *inputs):
        return inputs[0] * 2

    def run(self, config, *inputs):
        mode = config["MODE"]
        if mode == MODE_COMPILE:
            raise KernelNotCompiled("no instantiation")
        if mode == MODE_RUNTIME:
            raise RuntimeError("launch failed")
        if mode == MODE_OOM:
            raise FakeOutOfMemoryError("out of memory")
        if mode == MODE_WRONG:
            return inputs[0] * 3
        if mode == MODE_SLOW:
            time.sleep(0.002)
        return inputs[0] * 2

    def default_config(self, problem):
        return KernelConfig("fake", MODE=MODE_FAST)

    def flops(self, problem):
        return problem["n"]

    def bytes_moved(self, problem):
        return 8 * problem["n"]


def _tune(tmp_path, **kw):
    db = ResultsDB(tmp_path / "t.db")
    cache = ConfigCache(tmp_path / "c.json")
    tuner = Tuner(warmup=1, iterations=3, db=db, cache=cache, **kw)
    result = tuner.tune(_FakeOperator(), _problem(), device="cpu")
    return result, db, cache


def test_tuner_pipeline_on_cpu(tmp_path):
    result, db, cache = _tune(tmp_path)
    assert (result.generated, result.feasible, result.tested) == (7, 6, 6)
    statuses = {o.config["MODE"]: o.status for o in result.outcomes}
    assert statuses == {
        MODE_FAST: STATUS_OK,
        MODE_COMPILE: STATUS_COMPILE_ERROR,
        MODE_RUNTIME: STATUS_RUNTIME_ERROR,
        MODE_WRONG: STATUS_INCORRECT,
        MODE_SLOW: STATUS_OK,
        MODE_OOM: STATUS_OOM,
    }
    ranked = result.ranked()
    assert [o.config["MODE"] for o in ranked] == [MODE_FAST, MODE_SLOW]
    assert result.best_config == KernelConfig("fake", MODE=MODE_FAST)
    for o in result.outcomes:
        if not o.ok:
            assert o.timing is None and o.error
        else:
            assert o.timing.timer == "perf_counter"
    assert result.speedup_over("torch_eager") is not None
    # Persistence: every outcome plus the baseline is a row; the winner is cached.
    assert db.counts()["results"] == 6 + len(result.baselines)
    assert cache.get(_problem(), "cpu") == KernelConfig("fake", MODE=MODE_FAST)
    assert result.rejections and "infeasible" in result.rejections[0][1]


def test_tuner_budget_and_baselines_switch(tmp_path):
    result, _, _ = _tune(tmp_path, max_candidates=2, measure_baselines=False)
    assert result.tested == 2 and result.baselines == {}


def test_tuner_requires_a_gpu_by_default():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Tuner().tune(_FakeOperator(), _problem())


@pytest.mark.parametrize(
    "exc,status",
    [
        (type("KernelOutOfResources", (RuntimeError,), {})("lds"), STATUS_COMPILE_ERROR),
        (type("KernelNotCompiled", (RuntimeError,), {})("x"), STATUS_COMPILE_ERROR),
        (type("OutOfMemoryError", (RuntimeError,), {})("x"), STATUS_OOM),
        (ValueError("x"), STATUS_RUNTIME_ERROR),
    ],
)
def test_classify(exc, status):
    assert _classify(exc)[0] == status


def test_hip_error_classes_classify_as_the_tuner_expects():
    from kernelforge.runtime import hip

    assert _classify(hip.KernelNotCompiled("x"))[0] == STATUS_COMPILE_ERROR
    assert _classify(hip.KernelOutOfResources("x"))[0] == STATUS_COMPILE_ERROR
    assert _classify(hip.KernelOutOfMemoryError("x"))[0] == STATUS_OOM
    assert _classify(hip.KernelLaunchError("x"))[0] == STATUS_RUNTIME_ERROR


def test_shipped_config_is_a_device_lookup_only():
    """Off the GPU, and for empty shapes, an entry point without a configuration
    takes the heuristic: there is no shipped winner to look up."""
    import torch

    from kernelforge.runtime.dispatch import shipped_config

    assert shipped_config("matmul", torch.float16, torch.device("cpu"), M=2048, N=4096, K=4096) is None
    assert shipped_config("matmul", torch.float16, torch.device("cuda"), M=0, N=4096, K=4096) is None
