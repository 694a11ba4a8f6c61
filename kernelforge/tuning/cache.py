"""Persistent winner cache: ``device_key -> operation -> dtype -> shape_key``.

A serving process must not re-tune on start-up, so the winning configuration
is written to a JSON file and reused for an identical problem on an
identical device (kernelforge/tuning/cache.py:1-159). The device key is the
board name plus the architecture (``AMD_Instinct_MI355X_gfx950``), so a file
copied to other hardware misses instead of serving a foreign winner. Writes
go through a temporary file and ``os.replace``; an unknown version is
refused.
"""

from __future__ import annotations

import json
import os
import tempfile
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from kernelforge.tuning.config import KernelConfig, Problem

CACHE_VERSION = 1


#: Winners tuned on MI355X and shipped with the package; consulted by
#: dispatch after the user's cache, never written at run time.
PACKAGED_CACHE = Path(__file__).resolve().parent.parent / "tuned" / "mi355x_gfx950.json"


def default_cache_path() -> Path:
    for var in ("KERNELO_AMD_CACHE", "KERNELFORGE_CACHE"):
        if env := os.environ.get(var):
            return Path(env)
    root = Path(os.environ.get("XDG_CACHE_HOME", Path.home() / ".cache"))
    return root / "kernelforge" / "configs.json"


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
        params = ", ".join(f"{k}={v}" for k, v in self.config.as_dict().items())
        latency = f"{self.median_us:.1f} us" if self.median_us is not None else "unmeasured"
        return (
            f"{self.device_key}  {self.operation:<13} {self.dtype:<5} "
            f"{self.shape_key:<22} {latency:>12}  {params}"
        )


class ConfigCache:
    """A JSON file of best-known configurations."""

    def __init__(self, path: str | Path | None = None) -> None:
        self.path = Path(path) if path is not None else default_cache_path()
        self._data = self._load()

    def _load(self) -> dict[str, Any]:
        if not self.path.exists():
            return {"version": CACHE_VERSION, "entries": {}}
        try:
            data = json.loads(self.path.read_text())
        except json.JSONDecodeError as exc:
            raise RuntimeError(f"cache file {self.path} is not valid JSON: {exc}") from exc
        version = data.get("version") if isinstance(data, dict) else None
        if version != CACHE_VERSION:
            raise RuntimeError(
                f"cache file {self.path} has version {version}, expected {CACHE_VERSION}; "
                "run `kernelforge cache clear` to discard it"
            )
        return data

    def _flush(self) -> None:
        self.path.parent.mkdir(parents=True, exist_ok=True)
        fd, tmp = tempfile.mkstemp(dir=self.path.parent, suffix=".tmp")
        try:
            with os.fdopen(fd, "w") as handle:
                json.dump(self._data, handle, indent=2, sort_keys=True)
            os.replace(tmp, self.path)
        except BaseException:
            Path(tmp).unlink(missing_ok=True)
            raise

    def get(self, problem: Problem, device_key: str) -> KernelConfig | None:
        node = (
            self._data["entries"]
            .get(device_key, {})
            .get(problem.operation, {})
            .get(problem.dtype_name, {})
            .get(problem.shape_key)
        )
        if node is None:
            return None
        return KernelConfig(problem.operation, **node["config"])

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
        node = self._data["entries"].setdefault(device_key, {})
        node = node.setdefault(problem.operation, {})
        node = node.setdefault(problem.dtype_name, {})
        node[problem.shape_key] = {
            "config": config.as_dict(),
            "median_us": median_us,
            "timestamp": timestamp,
            "candidates_tested": candidates_tested,
        }
        self._flush()

    def entries(self) -> list[CacheEntry]:
        out: list[CacheEntry] = []
        for device_key, operations in self._data["entries"].items():
            for operation, dtypes in operations.items():
                for dtype, shapes in dtypes.items():
                    for shape_key, payload in shapes.items():
                        out.append(
                            CacheEntry(
                                device_key=device_key,
                                operation=operation,
                                dtype=dtype,
                                shape_key=shape_key,
                                config=KernelConfig(operation, **payload["config"]),
                                median_us=payload.get("median_us"),
                                timestamp=payload.get("timestamp", ""),
                                candidates_tested=payload.get("candidates_tested"),
                            )
                        )
        return sorted(out, key=lambda e: (e.device_key, e.operation, e.dtype, e.shape_key))

    def clear(self) -> int:
        removed = len(self.entries())
        self._data = {"version": CACHE_VERSION, "entries": {}}
        if self.path.exists():
            self.path.unlink()
        return removed

    def __len__(self) -> int:
        return len(self.entries())
