"""SQLite results store for tuning and benchmark runs.

Every result row points at the run that produced it (host, GPU, HIP, torch and
package versions), the problem, and the configuration, so a number from last
week stays comparable -- or visibly not -- with one from today. The tables are
the reference's (kernelforge/db.py:35-99), every column included, so a file
either tool created is read and written by the other: this build leaves
``triton_version`` and ``cuda_version`` empty, stores its compute-unit count in
``sm_count`` as well, and records what only it knows in two extra columns,
``hip_version`` and ``cu_count``. Opening a file the reference created adds
those two (nullable) columns; the reference names its columns in every
statement, so it keeps working on the widened table.

Here the schema is data: each table is a tuple of column declarations from
which the DDL and every INSERT are generated, so a column cannot be added to
one and forgotten in the other. Problems and configurations are interned
(insert-or-ignore on their natural key, then look the id up). A measurement is
flattened into columns by small per-part functions (timing, verification), and
a batch of measurements is one transaction. "Best per label" is one windowed
query. The schema version lives in ``PRAGMA user_version``; a file written by
another version is refused, not migrated.
"""

from __future__ import annotations

import json
import os
import sqlite3
from collections.abc import Iterable, Iterator
from contextlib import contextmanager
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Any

from kernelforge.runtime.env import Environment
from kernelforge.testing import VerificationResult
from kernelforge.tuning.config import KernelConfig, Problem

SCHEMA_VERSION = 1
DEFAULT_DB_PATH = Path("results/kernelforge.db")

_Columns = tuple[tuple[str, str], ...]

#: table -> (columns, table constraints); the first column is the row id.
_TABLES: dict[str, tuple[_Columns, tuple[str, ...]]] = {
    "runs": (
        (
            ("run_id", "INTEGER PRIMARY KEY AUTOINCREMENT"),
            ("timestamp", "TEXT NOT NULL"),
            ("hostname", "TEXT"),
            ("platform", "TEXT"),
            ("python_version", "TEXT"),
            ("torch_version", "TEXT"),
            ("triton_version", "TEXT"),
            ("cuda_version", "TEXT"),
            ("driver_version", "TEXT"),
            ("gpu_name", "TEXT"),
            ("gpu_arch", "TEXT"),
            ("gpu_memory_bytes", "INTEGER"),
            ("sm_count", "INTEGER"),
            ("device_key", "TEXT NOT NULL"),
            ("kernelforge_version", "TEXT"),
            ("notes", "TEXT NOT NULL DEFAULT ''"),
            # This build's own provenance, after the reference's columns.
            ("hip_version", "TEXT"),
            ("cu_count", "INTEGER"),
        ),
        (),
    ),
    "problems": (
        (
            ("problem_id", "INTEGER PRIMARY KEY AUTOINCREMENT"),
            ("operation", "TEXT NOT NULL"),
            ("shape_key", "TEXT NOT NULL"),
            ("dtype", "TEXT NOT NULL"),
            ("dims_json", "TEXT NOT NULL"),
        ),
        ("UNIQUE (operation, shape_key, dtype)",),
    ),
    "configs": (
        (
            ("config_id", "INTEGER PRIMARY KEY AUTOINCREMENT"),
            ("operation", "TEXT NOT NULL"),
            ("digest", "TEXT NOT NULL"),
            ("params_json", "TEXT NOT NULL"),
        ),
        ("UNIQUE (operation, digest)",),
    ),
    "results": (
        (
            ("result_id", "INTEGER PRIMARY KEY AUTOINCREMENT"),
            ("run_id", "INTEGER NOT NULL REFERENCES runs (run_id)"),
            ("problem_id", "INTEGER NOT NULL REFERENCES problems (problem_id)"),
            ("config_id", "INTEGER REFERENCES configs (config_id)"),
            ("label", "TEXT NOT NULL"),
            ("status", "TEXT NOT NULL"),
            ("correct", "INTEGER"),
            ("rel_error", "REAL"),
            ("median_us", "REAL"),
            ("mean_us", "REAL"),
            ("std_us", "REAL"),
            ("min_us", "REAL"),
            ("max_us", "REAL"),
            ("p95_us", "REAL"),
            ("p99_us", "REAL"),
            ("warmup", "INTEGER"),
            ("iterations", "INTEGER"),
            ("timer", "TEXT"),
            ("flushed_l2", "INTEGER"),
            ("tflops", "REAL"),
            ("gbps", "REAL"),
            ("error", "TEXT NOT NULL DEFAULT ''"),
        ),
        (),
    ),
}

_INDEXES = (
    "CREATE INDEX IF NOT EXISTS idx_results_problem ON results (problem_id, label)",
    "CREATE INDEX IF NOT EXISTS idx_results_run ON results (run_id)",
)


def _ddl() -> str:
    statements = []
    for table, (columns, constraints) in _TABLES.items():
        body = [f"{name} {decl}" for name, decl in columns] + list(constraints)
        statements.append(f"CREATE TABLE IF NOT EXISTS {table} ({', '.join(body)})")
    return ";\n".join(statements + list(_INDEXES)) + ";"


def _insertable(table: str) -> tuple[str, ...]:
    """Columns an INSERT names: all but the auto-assigned id."""
    return tuple(name for name, _ in _TABLES[table][0][1:])


#: The joined view every read returns: result, problem, config and run provenance.
_JOINED = {
    "r": ("result_id", "label", "status", "correct", "rel_error", "median_us", "mean_us", "std_us",
          "min_us", "max_us", "p95_us", "p99_us", "warmup", "iterations", "timer", "flushed_l2",
          "tflops", "gbps", "error"),
    "p": ("operation", "shape_key", "dtype", "dims_json"),
    "c": ("params_json", "digest"),
    "run": ("run_id", "timestamp", "gpu_name", "gpu_arch", "device_key", "torch_version",
            "triton_version", "cuda_version", "driver_version", "hip_version"),
}
_FROM = ("FROM results AS r JOIN problems AS p ON p.problem_id = r.problem_id "
         "JOIN runs AS run ON run.run_id = r.run_id "
         "LEFT JOIN configs AS c ON c.config_id = r.config_id")
_SELECT = "SELECT " + ", ".join(f"{alias}.{col}" for alias, cols in _JOINED.items() for col in cols)


@dataclass(frozen=True)
class Measurement:
    """One row to record: what ran, whether it was right, and how fast."""

    label: str
    status: str
    config: KernelConfig | None = None
    verification: VerificationResult | None = None
    timing: Any = None  # a TimingResult; typed loosely so this module needs no GPU imports
    tflops: float | None = None
    gbps: float | None = None
    error: str = ""


def _timing_columns(timing: Any) -> dict[str, Any]:
    stats_us = ("median", "mean", "std", "min", "max", "p95", "p99")
    if timing is None:
        return {**{f"{s}_us": None for s in stats_us},
                "warmup": None, "iterations": None, "timer": None, "flushed_l2": None}
    out: dict[str, Any] = {f"{s}_us": getattr(timing, f"{s}_ms") * 1e3 for s in stats_us}
    out.update(warmup=timing.warmup, iterations=timing.iterations, timer=timing.timer,
               flushed_l2=int(bool(timing.flushed_l2)))
    return out


def _verification_columns(result: VerificationResult | None) -> dict[str, Any]:
    if result is None:
        return {"correct": None, "rel_error": None}
    return {"correct": int(result.passed), "rel_error": result.error}


def default_db_path() -> Path:
    """``$KERNELFORGE_DB``, else ``results/kernelforge.db`` under the working directory."""
    return Path(os.environ.get("KERNELFORGE_DB") or DEFAULT_DB_PATH)


class ResultsDB:
    """The results database behind ``tune``, ``benchmark``, ``compare`` and ``report``."""

    def __init__(self, path: str | Path | None = None) -> None:
        self.path = Path(path) if path is not None else default_db_path()
        in_memory = str(self.path) == ":memory:"
        if not in_memory:
            self.path.parent.mkdir(parents=True, exist_ok=True)
        self._conn = sqlite3.connect(str(self.path))
        self._conn.row_factory = sqlite3.Row
        self._conn.execute("PRAGMA foreign_keys = ON")
        version = int(self._conn.execute("PRAGMA user_version").fetchone()[0])
        if version not in (0, SCHEMA_VERSION):
            self._conn.close()
            raise RuntimeError(
                f"{self.path} was written by schema version {version}, "
                f"this build expects {SCHEMA_VERSION}"
            )
        with self._conn:
            self._conn.executescript(_ddl())
            self._widen()
            self._conn.execute(f"PRAGMA user_version = {SCHEMA_VERSION}")

    def _widen(self) -> None:
        """Add the columns of this build's schema an existing table lacks (a file
        the reference created has no ``hip_version`` or ``cu_count``). Only
        nullable columns can be missing; anything else is a foreign schema."""
        for table, (columns, _) in _TABLES.items():
            have = {row[1] for row in self._conn.execute(f"PRAGMA table_info({table})")}
            for name, decl in columns:
                if name in have:
                    continue
                if "NOT NULL" in decl or "PRIMARY KEY" in decl:
                    raise RuntimeError(f"{self.path}: table {table} has no column {name}; "
                                       "not a kernelforge results database")
                self._conn.execute(f"ALTER TABLE {table} ADD COLUMN {name} {decl}")

    def __enter__(self) -> ResultsDB:
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def close(self) -> None:
        self._conn.close()

    # --- writes -------------------------------------------------------------------
    @contextmanager
    def _transaction(self) -> Iterator[sqlite3.Connection]:
        with self._conn:  # commits on success, rolls back on error
            yield self._conn

    def _insert(self, table: str, values: dict[str, Any]) -> int:
        names = [c for c in _insertable(table) if c in values]
        sql = f"INSERT INTO {table} ({', '.join(names)}) VALUES ({', '.join('?' * len(names))})"
        return int(self._conn.execute(sql, [values[c] for c in names]).lastrowid)

    def _intern(self, table: str, natural_key: dict[str, Any], extra: dict[str, Any]) -> int:
        """Id of the row with ``natural_key``, inserting it (with ``extra``) if new."""
        id_col = _TABLES[table][0][0][0]
        names = list(natural_key) + list(extra)
        self._conn.execute(
            f"INSERT OR IGNORE INTO {table} ({', '.join(names)}) "
            f"VALUES ({', '.join('?' * len(names))})",
            [*natural_key.values(), *extra.values()],
        )
        where = " AND ".join(f"{k} = ?" for k in natural_key)
        row = self._conn.execute(f"SELECT {id_col} FROM {table} WHERE {where}",
                                 list(natural_key.values())).fetchone()
        return int(row[0])

    def start_run(self, env: Environment, *, notes: str = "", version: str = "") -> int:
        """Record the environment of a run; its id tags every result of that run."""
        values = {k: v for k, v in asdict(env).items() if k in _insertable("runs")}
        # No Triton and no CUDA here; the reference's SM-count column gets the
        # compute-unit count, its nearest counterpart.
        values.update(triton_version=None, cuda_version=None, sm_count=env.cu_count,
                      kernelforge_version=version, notes=notes)
        with self._transaction():
            return self._insert("runs", values)

    def problem_id(self, problem: Problem) -> int:
        with self._transaction():
            return self._intern(
                "problems",
                {"operation": problem.operation, "shape_key": problem.shape_key,
                 "dtype": problem.dtype_name},
                {"dims_json": json.dumps(problem.dims_dict, sort_keys=True)},
            )

    def config_id(self, config: KernelConfig) -> int:
        with self._transaction():
            return self._intern("configs", {"operation": config.operation, "digest": config.digest},
                                {"params_json": config.to_json()})

    def _result(self, run_id: int, problem_id: int, m: Measurement) -> int:
        config_id = None
        if m.config is not None:
            config_id = self._intern("configs", {"operation": m.config.operation,
                                                 "digest": m.config.digest},
                                     {"params_json": m.config.to_json()})
        values = {"run_id": run_id, "problem_id": problem_id, "config_id": config_id,
                  "label": m.label, "status": m.status, "tflops": m.tflops, "gbps": m.gbps,
                  "error": m.error}
        values.update(_verification_columns(m.verification))
        values.update(_timing_columns(m.timing))
        return self._insert("results", values)

    def record_many(self, run_id: int, problem: Problem, measurements: Iterable[Measurement]) -> list[int]:
        """Record several measurements of one problem in one transaction."""
        pid = self.problem_id(problem)
        with self._transaction():
            return [self._result(run_id, pid, m) for m in measurements]

    def record(self, run_id: int, problem: Problem, measurement: Measurement) -> int:
        return self.record_many(run_id, problem, [measurement])[0]

    # --- reads --------------------------------------------------------------------
    def _select(self, where: dict[str, str | None], tail: str) -> list[dict]:
        active = {col: val for col, val in where.items() if val}
        sql = f"{_SELECT} {_FROM}"
        if active:
            sql += " WHERE " + " AND ".join(f"{col} = ?" for col in active)
        return [dict(r) for r in self._conn.execute(f"{sql} {tail}", list(active.values()))]

    def rows(self, *, operation: str | None = None, dtype: str | None = None) -> list[dict]:
        """Every result joined with its problem, config and run, in insertion order."""
        return self._select({"p.operation": operation, "p.dtype": dtype}, "ORDER BY r.result_id")

    def best_per_label(self, *, operation: str | None = None) -> list[dict]:
        """The fastest timed, not-incorrect result of each (problem, label).

        Rows without a timing or whose verification failed never win; ties go
        to the earlier row.
        """
        ranked = (
            f"{_SELECT}, ROW_NUMBER() OVER (PARTITION BY r.problem_id, r.label "
            f"ORDER BY r.median_us, r.result_id) AS rank_in_label {_FROM} "
            "WHERE r.median_us IS NOT NULL AND (r.correct IS NULL OR r.correct != 0)"
        )
        args: list[str] = []
        if operation:
            ranked += " AND p.operation = ?"
            args.append(operation)
        sql = (f"SELECT * FROM ({ranked}) WHERE rank_in_label = 1 "
               "ORDER BY operation, dtype, shape_key, label")
        out = [dict(r) for r in self._conn.execute(sql, args)]
        for row in out:
            row.pop("rank_in_label")
        return out

    def runs(self) -> list[dict]:
        """Every recorded run, oldest first, including runs that recorded nothing."""
        return [dict(r) for r in self._conn.execute("SELECT * FROM runs ORDER BY run_id")]

    def counts(self) -> dict[str, int]:
        return {t: int(self._conn.execute(f"SELECT COUNT(*) FROM {t}").fetchone()[0])
                for t in _TABLES}

    def operations(self) -> list[str]:
        return [r[0] for r in self._conn.execute(
            "SELECT DISTINCT operation FROM problems ORDER BY operation")]
