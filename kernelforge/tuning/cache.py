"""The JSON winner cache: best-known configuration per device, op, dtype and shape.

Tuning costs minutes; a serving process reads its winners from this file in
microseconds and never tunes (kernelforge/tuning/cache.py:1-159). The file
format is the reference's, so cache files move between the two tools::

    {"version": 1,
     "entries": {<device key>: {<operation>: {<dtype>: {<shape key>:
         {"config": {...}, "median_us": ..., "timestamp": ..., "candidates_tested": ...}}}}}}

The device key is the board plus the architecture
(``AMD_Instinct_MI355X_gfx950``): a file copied to other hardware misses rather
than serving a winner tuned elsewhere.

In memory the nesting is flattened to one index keyed by
``(device, operation, dtype, shape)``; the nested form exists only on disk.
Every change is written through a temporary file in the same directory and
``os.replace``, so a reader never sees a half-written file. Two files are
consulted by dispatch: the user's (read-write) and the winners packaged with
this build (read-only).
"""

from __future__ import annotations

import json
import os
import tempfile
from dataclasses import dataclass
from pathlib import Path
from typing import Any, NamedTuple

from kernelforge.tuning.config import KernelConfig, Problem

CACHE_VERSION = 1

#: Winners tuned on MI355X and shipped with the package; dispatch consults them
#: after the user's cache and nothing writes them at run time.
PACKAGED_CACHE = Path(__file__).resolve().parent.parent / "tuned" / "mi355x_gfx950.json"


def default_cache_path() -> Path:
    """``$KERNELFORGE_CACHE``, else ``$XDG_CACHE_HOME/kernelforge/configs.json``."""
    explicit = os.environ.get("KERNELFORGE_CACHE")
    if explicit:
        return Path(explicit)
    base = os.environ.get("XDG_CACHE_HOME") or str(Path.home() / ".cache")
    return Path(base) / "kernelforge" / "configs.json"


class _Key(NamedTuple):
    device_key: str
    operation: str
    dtype: str
    shape_key: str


@dataclass(frozen=True)
class CacheEntry:
    device_key: str
    operation: str
    dtype: str
    shape_key: str
    config: KernelConfig
    median_us: float | None
    timestamp: str
    candidates_tested: int | None = None

    def describe(self) -> str:
        """One aligned line for ``kernelforge cache list``."""
        took = "unmeasured" if self.median_us is None else f"{self.median_us:.1f} us"
        params = ", ".join(f"{k}={v}" for k, v in self.config.items())
        return (f"{self.device_key}  {self.operation:<13} {self.dtype:<5} {self.shape_key:<22} "
                f"{took:>12}  {params}")


def _flatten(document: dict[str, Any]) -> dict[_Key, dict[str, Any]]:
    flat: dict[_Key, dict[str, Any]] = {}
    for device, per_op in document.get("entries", {}).items():
        for operation, per_dtype in per_op.items():
            for dtype, per_shape in per_dtype.items():
                for shape, record in per_shape.items():
                    flat[_Key(device, operation, dtype, shape)] = record
    return flat


def _nest(flat: dict[_Key, dict[str, Any]]) -> dict[str, Any]:
    entries: dict[str, Any] = {}
    for key in sorted(flat):
        level = entries
        for part in key[:-1]:
            level = level.setdefault(part, {})
        level[key.shape_key] = flat[key]
    return {"version": CACHE_VERSION, "entries": entries}


class ConfigCache:
    """One winner file. ``read_only`` caches refuse ``put`` and ``clear``."""

    def __init__(self, path: str | Path | None = None, *, read_only: bool = False) -> None:
        self.path = Path(path) if path is not None else default_cache_path()
        self.read_only = read_only
        self._records = self._read()

    def _read(self) -> dict[_Key, dict[str, Any]]:
        try:
            text = self.path.read_text()
        except FileNotFoundError:
            return {}
        try:
            document = json.loads(text)
        except json.JSONDecodeError as exc:
            raise RuntimeError(f"cache file {self.path} is not valid JSON: {exc}") from exc
        found = document.get("version") if isinstance(document, dict) else None
        if found != CACHE_VERSION:
            raise RuntimeError(
                f"cache file {self.path} has version {found}, expected {CACHE_VERSION}; "
                "run `kernelforge cache clear` to discard it"
            )
        return _flatten(document)

    def _write(self) -> None:
        self.path.parent.mkdir(parents=True, exist_ok=True)
        payload = json.dumps(_nest(self._records), indent=2, sort_keys=True)
        handle = tempfile.NamedTemporaryFile(
            "w", dir=self.path.parent, prefix=f".{self.path.name}.", suffix=".tmp", delete=False
        )
        try:
            with handle:
                handle.write(payload)
                handle.flush()
                os.fsync(handle.fileno())
            os.replace(handle.name, self.path)
        except BaseException:
            Path(handle.name).unlink(missing_ok=True)
            raise

    def _guard(self, what: str) -> None:
        if self.read_only:
            raise PermissionError(f"{self.path} is a read-only winner file; cannot {what}")

    @staticmethod
    def _key(problem: Problem, device_key: str) -> _Key:
        return _Key(device_key, problem.operation, problem.dtype_name, problem.shape_key)

    def get(self, problem: Problem, device_key: str) -> KernelConfig | None:
        record = self._records.get(self._key(problem, device_key))
        return None if record is None else KernelConfig(problem.operation, **record["config"])

    def put(
        self,
        problem: Problem,
        device_key: str,
        config: KernelConfig,
        *,
        median_us: float | None = None,
        timestamp: str = "",
        candidates_tested: int | None = None,
    ) -> None:
        self._guard("store a winner")
        self._records[self._key(problem, device_key)] = {
            "config": config.as_dict(),
            "median_us": median_us,
            "timestamp": timestamp,
            "candidates_tested": candidates_tested,
        }
        self._write()

    def entries(self) -> list[CacheEntry]:
        return [
            CacheEntry(
                device_key=key.device_key,
                operation=key.operation,
                dtype=key.dtype,
                shape_key=key.shape_key,
                config=KernelConfig(key.operation, **record["config"]),
                median_us=record.get("median_us"),
                timestamp=record.get("timestamp", ""),
                candidates_tested=record.get("candidates_tested"),
            )
            for key, record in sorted(self._records.items())
        ]

    def clear(self) -> int:
        """Forget every entry and delete the file; returns how many there were."""
        self._guard("clear it")
        count = len(self._records)
        self._records = {}
        self.path.unlink(missing_ok=True)
        return count

    def __len__(self) -> int:
        return len(self._records)
