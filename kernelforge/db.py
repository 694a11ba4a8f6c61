"""SQLite store for tuning and benchmark results.

Same role and schema shape as the reference (kernelforge/db.py:35-320): runs
carry provenance, problems and configs are deduplicated (configs by their
JSON parameter set and digest), and results point at all three. Columns name
what this build records: ``hip_version`` and ``cu_count`` where the reference
stored CUDA/Triton versions and an SM count. The schema version lives in
``PRAGMA user_version`` and a mismatch is refused rather than migrated.
"""

from __future__ import annotations

import json
import os
import sqlite3
from collections.abc import Iterable
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from kernelforge.runtime.env import Environment
from kernelforge.testing import VerificationResult
from kernelforge.tuning.config import KernelConfig, Problem

SCHEMA_VERSION = 1
DEFAULT_DB_PATH = Path("results/kernelforge.db")

_SCHEMA = """
CREATE TABLE IF NOT EXISTS runs (
    run_id              INTEGER PRIMARY KEY AUTOINCREMENT,
    timestamp           TEXT    NOT NULL,
    hostname            TEXT,
    platform            TEXT,
    python_version      TEXT,
    torch_version       TEXT,
    hip_version         TEXT,
    driver_version      TEXT,
    gpu_name            TEXT,
    gpu_arch            TEXT,
    gpu_memory_bytes    INTEGER,
    cu_count            INTEGER,
    device_key          TEXT    NOT NULL,
    package_version     TEXT,
    notes               TEXT    NOT NULL DEFAULT ''
);

CREATE TABLE IF NOT EXISTS problems (
    problem_id INTEGER PRIMARY KEY AUTOINCREMENT,
    operation  TEXT NOT NULL,
    shape_key  TEXT NOT NULL,
    dtype      TEXT NOT NULL,
    dims_json  TEXT NOT NULL,
    UNIQUE (operation, shape_key, dtype)
);

CREATE TABLE IF NOT EXISTS configs (
    config_id   INTEGER PRIMARY KEY AUTOINCREMENT,
    operation   TEXT NOT NULL,
    digest      TEXT NOT NULL,
    params_json TEXT NOT NULL,
    UNIQUE (operation, digest)
);

CREATE TABLE IF NOT EXISTS results (
    result_id  INTEGER PRIMARY KEY AUTOINCREMENT,
    run_id     INTEGER NOT NULL REFERENCES runs (run_id),
    problem_id INTEGER NOT NULL REFERENCES problems (problem_id),
    config_id  INTEGER          REFERENCES configs (config_id),
    label      TEXT    NOT NULL,
    status     TEXT    NOT NULL,
    correct    INTEGER,
    rel_error  REAL,
    median_us  REAL,
    mean_us    REAL,
    std_us     REAL,
    min_us     REAL,
    max_us     REAL,
    p95_us     REAL,
    p99_us     REAL,
    warmup     INTEGER,
    iterations INTEGER,
    timer      TEXT,
    flushed_l2 INTEGER,
    tflops     REAL,
    gbps       REAL,
    error      TEXT NOT NULL DEFAULT ''
);

CREATE INDEX IF NOT EXISTS idx_results_problem ON results (problem_id, label);
CREATE INDEX IF NOT EXISTS idx_results_run     ON results (run_id);
"""

_ROWS_QUERY = """
SELECT
    r.result_id, r.label, r.status, r.correct, r.rel_error,
    r.median_us, r.mean_us, r.std_us, r.min_us, r.max_us, r.p95_us, r.p99_us,
    r.warmup, r.iterations, r.timer, r.flushed_l2, r.tflops, r.gbps, r.error,
    p.operation, p.shape_key, p.dtype, p.dims_json,
    c.params_json, c.digest,
    run.run_id, run.timestamp, run.gpu_name, run.gpu_arch, run.device_key,
    run.torch_version, run.hip_version, run.driver_version
FROM results AS r
JOIN problems AS p   ON p.problem_id = r.problem_id
JOIN runs     AS run ON run.run_id   = r.run_id
LEFT JOIN configs AS c ON c.config_id = r.config_id
"""


@dataclass(frozen=True)
class Measurement:
    """One row to record: what ran, whether it was right, and how fast."""

    label: str
    status: str
    config: KernelConfig | None = None
    verification: VerificationResult | None = None
    timing: Any = None  # TimingResult (kept loose so this module stays import-light)
    tflops: float | None = None
    gbps: float | None = None
    error: str = ""


def default_db_path() -> Path:
    return Path(os.environ.get("KERNELO_AMD_DB", os.environ.get("KERNELFORGE_DB", DEFAULT_DB_PATH)))


class ResultsDB:
    """Explicit wrapper over the results database."""

    def __init__(self, path: str | Path | None = None) -> None:
        self.path = Path(path) if path is not None else default_db_path()
        if str(self.path) != ":memory:":
            self.path.parent.mkdir(parents=True, exist_ok=True)
        self._conn = sqlite3.connect(str(self.path))
        self._conn.row_factory = sqlite3.Row
        self._conn.execute("PRAGMA foreign_keys = ON")
        self._conn.executescript(_SCHEMA)
        self._check_schema_version()
        self._conn.commit()

    def _check_schema_version(self) -> None:
        current = int(self._conn.execute("PRAGMA user_version").fetchone()[0])
        if current == 0:
            self._conn.execute(f"PRAGMA user_version = {SCHEMA_VERSION}")
        elif current != SCHEMA_VERSION:
            raise RuntimeError(
                f"{self.path} was written by schema version {current}, "
                f"this build expects {SCHEMA_VERSION}"
            )

    def __enter__(self) -> ResultsDB:
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def close(self) -> None:
        self._conn.close()

    # --- writes ---------------------------------------------------------------
    def start_run(self, env: Environment, *, notes: str = "", version: str = "") -> int:
        cur = self._conn.execute(
            """
            INSERT INTO runs (
                timestamp, hostname, platform, python_version, torch_version, hip_version,
                driver_version, gpu_name, gpu_arch, gpu_memory_bytes, cu_count, device_key,
                package_version, notes
            ) VALUES (?,?,?,?,?,?,?,?,?,?,?,?,?,?)
            """,
            (
                env.timestamp,
                env.hostname,
                env.platform,
                env.python_version,
                env.torch_version,
                env.hip_version,
                env.driver_version,
                env.gpu_name,
                env.gpu_arch,
                env.gpu_memory_bytes,
                env.cu_count,
                env.device_key,
                version,
                notes,
            ),
        )
        self._conn.commit()
        return int(cur.lastrowid)

    def problem_id(self, problem: Problem) -> int:
        self._conn.execute(
            "INSERT OR IGNORE INTO problems (operation, shape_key, dtype, dims_json) "
            "VALUES (?,?,?,?)",
            (
                problem.operation,
                problem.shape_key,
                problem.dtype_name,
                json.dumps(problem.dims_dict, sort_keys=True),
            ),
        )
        row = self._conn.execute(
            "SELECT problem_id FROM problems WHERE operation=? AND shape_key=? AND dtype=?",
            (problem.operation, problem.shape_key, problem.dtype_name),
        ).fetchone()
        return int(row["problem_id"])

    def config_id(self, config: KernelConfig) -> int:
        self._conn.execute(
            "INSERT OR IGNORE INTO configs (operation, digest, params_json) VALUES (?,?,?)",
            (config.operation, config.digest, config.to_json()),
        )
        row = self._conn.execute(
            "SELECT config_id FROM configs WHERE operation=? AND digest=?",
            (config.operation, config.digest),
        ).fetchone()
        return int(row["config_id"])

    def record(self, run_id: int, problem: Problem, measurement: Measurement) -> int:
        t = measurement.timing
        v = measurement.verification
        us = (lambda ms: None if t is None else ms * 1e3)
        cur = self._conn.execute(
            """
            INSERT INTO results (
                run_id, problem_id, config_id, label, status, correct, rel_error,
                median_us, mean_us, std_us, min_us, max_us, p95_us, p99_us,
                warmup, iterations, timer, flushed_l2, tflops, gbps, error
            ) VALUES (?,?,?,?,?,?,?,?,?,?,?,?,?,?,?,?,?,?,?,?,?)
            """,
            (
                run_id,
                self.problem_id(problem),
                self.config_id(measurement.config) if measurement.config is not None else None,
                measurement.label,
                measurement.status,
                None if v is None else int(v.passed),
                None if v is None else v.error,
                us(t.median_ms) if t else None,
                us(t.mean_ms) if t else None,
                us(t.std_ms) if t else None,
                us(t.min_ms) if t else None,
                us(t.max_ms) if t else None,
                us(t.p95_ms) if t else None,
                us(t.p99_ms) if t else None,
                None if t is None else t.warmup,
                None if t is None else t.iterations,
                None if t is None else t.timer,
                None if t is None else int(t.flushed_l2),
                measurement.tflops,
                measurement.gbps,
                measurement.error,
            ),
        )
        self._conn.commit()
        return int(cur.lastrowid)

    def record_many(self, run_id: int, problem: Problem, measurements: Iterable[Measurement]) -> None:
        for m in measurements:
            self.record(run_id, problem, m)

    # --- reads ----------------------------------------------------------------
    def rows(self, *, operation: str | None = None, dtype: str | None = None) -> list[dict]:
        clauses, params = [], []
        if operation:
            clauses.append("p.operation = ?")
            params.append(operation)
        if dtype:
            clauses.append("p.dtype = ?")
            params.append(dtype)
        query = _ROWS_QUERY
        if clauses:
            query += " WHERE " + " AND ".join(clauses)
        query += " ORDER BY r.result_id"
        return [dict(row) for row in self._conn.execute(query, params)]

    def best_per_label(self, *, operation: str | None = None) -> list[dict]:
        """Fastest correct measurement for each (problem, label) pair."""
        best: dict[tuple[str, str, str, str], dict] = {}
        for row in self.rows(operation=operation):
            if row["median_us"] is None or row["correct"] == 0:
                continue
            key = (row["operation"], row["shape_key"], row["dtype"], row["label"])
            if key not in best or row["median_us"] < best[key]["median_us"]:
                best[key] = row
        return sorted(
            best.values(), key=lambda r: (r["operation"], r["dtype"], r["shape_key"], r["label"])
        )

    def runs(self) -> list[dict]:
        """Every recorded run, oldest first (including runs that recorded nothing)."""
        return [dict(row) for row in self._conn.execute("SELECT * FROM runs ORDER BY run_id")]

    def counts(self) -> dict[str, int]:
        tables = ("runs", "problems", "configs", "results")
        return {t: int(self._conn.execute(f"SELECT COUNT(*) FROM {t}").fetchone()[0]) for t in tables}

    def operations(self) -> list[str]:
        return [r[0] for r in self._conn.execute("SELECT DISTINCT operation FROM problems ORDER BY 1")]
