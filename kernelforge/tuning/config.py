"""Descriptors: what is being run (``Problem``) and how (``KernelConfig``).

On this build a configuration does not parameterise a JIT compile; it names
one ahead-of-time instantiation in ``libkernelforge_hip.so`` (tile shape,
pipeline, stage count) plus the launch arguments the C-ABI takes for it
(waves per workgroup, split-K, group size). Configurations stay open integer
mappings, because the row kernels, the GEMV and the GEMM tiles have disjoint
parameter sets.

The interchange formats are the reference's, so results databases and cache
files stay readable by either tool (kernelforge/tuning/config.py:33-150):

* canonical JSON: keys sorted, no whitespace (``{"BLOCK_M":64,"num_warps":8}``);
* digest: the first 16 hex digits of sha1 over ``"<operation>|<json>"``;
* shape key: dimension values joined by ``x`` in declaration order, and the
  cache key ``<operation>/<dtype>/<shape key>``.

``num_warps`` counts 64-lane wavefronts and ``num_stages`` LDS buffers; they
are the launch keys, everything else picks the instantiation.
"""

from __future__ import annotations

import hashlib
import json
from collections.abc import Iterator, Mapping
from typing import Any

import torch

from kernelforge.dtypes import dtype_name, itemsize, parse_dtype

#: Keys that describe the launch rather than the instantiation (config.py:30).
LAUNCH_KEYS = frozenset({"num_warps", "num_stages"})


def _canonical(params: Mapping[str, int]) -> str:
    return json.dumps(dict(params), sort_keys=True, separators=(",", ":"))


def _require_int(key: str, value: object) -> int:
    # bool is an int subclass and numpy integers are not ints: both are refused,
    # so a config always serialises to plain JSON integers.
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"config parameter {key!r} must be an int, got {value!r}")
    return int(value)


def _rebuild_config(operation: str, pairs: tuple[tuple[str, int], ...]) -> KernelConfig:
    return KernelConfig(operation, **dict(pairs))


class KernelConfig(Mapping[str, int]):
    """Immutable, hashable, order-independent integer parameters of one operation.

    Stored as a sorted tuple of pairs; the mapping view, the canonical JSON
    and the digest are all derived from it, so two configs are equal exactly
    when their digests are.
    """

    __slots__ = ("operation", "_pairs", "_index")

    def __init__(self, operation: str, **params: int) -> None:
        pairs = tuple(sorted((k, _require_int(k, v)) for k, v in params.items()))
        object.__setattr__(self, "operation", operation)
        object.__setattr__(self, "_pairs", pairs)
        object.__setattr__(self, "_index", dict(pairs))

    def __setattr__(self, name: str, value: object) -> None:
        raise AttributeError("KernelConfig is immutable; use with_params()")

    def __reduce__(self):
        return (_rebuild_config, (self.operation, self._pairs))

    # Mapping protocol ------------------------------------------------------
    def __getitem__(self, key: str) -> int:
        return self._index[key]

    def __iter__(self) -> Iterator[str]:
        return (k for k, _ in self._pairs)

    def __len__(self) -> int:
        return len(self._pairs)

    def __hash__(self) -> int:
        return hash((self.operation, self._pairs))

    def __eq__(self, other: object) -> bool:
        if isinstance(other, KernelConfig):
            return (self.operation, self._pairs) == (other.operation, other._pairs)
        return NotImplemented

    def __repr__(self) -> str:
        inner = ", ".join(f"{k}={v}" for k, v in self._pairs)
        return f"KernelConfig({self.operation!r}, {inner})"

    # Views ------------------------------------------------------------------
    def _split(self, launch: bool) -> dict[str, int]:
        return {k: v for k, v in self._pairs if (k in LAUNCH_KEYS) == launch}

    @property
    def meta(self) -> dict[str, int]:
        """Instantiation parameters: tile, pipeline, split and strip sizes."""
        return self._split(launch=False)

    @property
    def launch(self) -> dict[str, int]:
        """Launch parameters: ``num_warps`` (wave64 count) and ``num_stages``."""
        return self._split(launch=True)

    @property
    def waves(self) -> int | None:
        """Wavefronts per workgroup (``num_warps``), if the config sets it."""
        return self._index.get("num_warps")

    def as_dict(self) -> dict[str, int]:
        return dict(self._pairs)

    def with_params(self, **changes: int) -> KernelConfig:
        """A copy with some parameters replaced or added."""
        merged = dict(self._pairs)
        merged.update(changes)
        return KernelConfig(self.operation, **merged)

    # Interchange --------------------------------------------------------------
    def to_json(self) -> str:
        return _canonical(self._index)

    @property
    def digest(self) -> str:
        """Database identity: sha1 of ``operation|canonical json``, 16 hex digits."""
        return hashlib.sha1(f"{self.operation}|{self.to_json()}".encode()).hexdigest()[:16]

    @classmethod
    def from_json(cls, operation: str, payload: str) -> KernelConfig:
        return cls(operation, **json.loads(payload))

    @classmethod
    def parse(cls, operation: str, text: str) -> KernelConfig:
        """``"BLOCK_M=128,BLOCK_N=256,num_warps=8"`` (the CLI's --config form)."""
        params: dict[str, int] = {}
        for item in filter(None, (part.strip() for part in text.split(","))):
            key, sep, value = item.partition("=")
            if not sep:
                raise ValueError(f"config item {item!r} is not KEY=VALUE")
            params[key.strip()] = int(value)
        return cls(operation, **params)

    def render(self, order: tuple[str, ...] = ()) -> str:
        """One ``KEY: value`` line per parameter, keys in ``order`` first, aligned."""
        ranked = sorted(self._index, key=lambda k: (order.index(k) if k in order else len(order), k))
        pad = 1 + max((len(k) for k in ranked), default=0)
        return "\n".join(f"{(k + ':').ljust(pad)} {self._index[k]:>4}" for k in ranked)


#: Operand layouts a product's problem can name. ``""`` is B stored (K, N)
#: row-major, the reference's only case; ``"bt"`` is B read k-contiguous, an
#: ``nn.Linear`` weight passed as ``weight.t()``. The decode GEMV runs a
#: different kernel for each (a column's k-run is contiguous only in the
#: second), so their tuned configurations are kept apart.
LAYOUTS = ("", "bt")
_LAYOUT_OPERATIONS = ("matmul", "fused_linear")


class Problem:
    """One workload: an operation over named dimensions in one dtype.

    Dimension names travel with the values (``M/N/K`` for products,
    ``rows/cols`` for row kernels, ``n`` for elementwise) because they become
    parts of cache keys and database rows. A product over k-contiguous B
    carries ``layout="bt"``, which its keys show as a ``+bt`` suffix; every
    other problem's keys are the reference's.
    """

    __slots__ = ("operation", "dims", "dtype", "layout", "_key")

    def __init__(self, operation: str, dims: tuple[tuple[str, int], ...], dtype: torch.dtype,
                 layout: str = ""):
        if layout not in LAYOUTS:
            raise ValueError(f"unknown operand layout {layout!r}; expected one of {LAYOUTS}")
        if layout and operation not in _LAYOUT_OPERATIONS:
            raise ValueError(f"{operation} has no operand layouts")
        object.__setattr__(self, "operation", operation)
        object.__setattr__(self, "dims", tuple((str(k), int(v)) for k, v in dims))
        object.__setattr__(self, "dtype", dtype)
        object.__setattr__(self, "layout", layout)
        object.__setattr__(self, "_key", (operation, self.dims, dtype, layout))

    def __setattr__(self, name: str, value: object) -> None:
        raise AttributeError("Problem is immutable")

    def __reduce__(self):
        return (Problem, (self.operation, self.dims, self.dtype, self.layout))

    @classmethod
    def create(cls, operation: str, dtype: str | torch.dtype, *, layout: str = "",
               **dims: int) -> Problem:
        bad = {k: v for k, v in dims.items() if isinstance(v, bool) or not isinstance(v, int) or v < 1}
        if bad:
            key, value = next(iter(bad.items()))
            raise ValueError(f"dimension {key!r} must be a positive int, got {value!r}")
        return cls(operation, tuple(dims.items()), parse_dtype(dtype), layout)

    def with_layout(self, layout: str) -> Problem:
        return Problem(self.operation, self.dims, self.dtype, layout)

    def __eq__(self, other: object) -> bool:
        if isinstance(other, Problem):
            return self._key == other._key
        return NotImplemented

    def __hash__(self) -> int:
        return hash(self._key)

    def __repr__(self) -> str:
        return f"Problem({self.cache_key})"

    def __getitem__(self, key: str) -> int:
        for name, value in self.dims:
            if name == key:
                return value
        raise KeyError(key)

    @property
    def dims_dict(self) -> dict[str, int]:
        return dict(self.dims)

    @property
    def shape_key(self) -> str:
        """Values in declaration order: ``2048x4096x4096`` (``1x11008x4096+bt``)."""
        key = "x".join(map(str, (v for _, v in self.dims)))
        return f"{key}+{self.layout}" if self.layout else key

    @property
    def dtype_name(self) -> str:
        return dtype_name(self.dtype)

    @property
    def itemsize(self) -> int:
        return itemsize(self.dtype)

    @property
    def cache_key(self) -> str:
        return "/".join((self.operation, self.dtype_name, self.shape_key))

    def describe(self) -> str:
        """``matmul M/N/K=2048 x 4096 x 4096 fp16``."""
        names = "/".join(name for name, _ in self.dims)
        values = " x ".join(str(v) for _, v in self.dims)
        tail = ", B k-contiguous" if self.layout == "bt" else ""
        return f"{self.operation} {names}={values} {self.dtype_name}{tail}"

    def as_dict(self) -> dict[str, Any]:
        out = {"operation": self.operation, "dims": self.dims_dict, "dtype": self.dtype_name,
               "shape_key": self.shape_key}
        if self.layout:
            out["layout"] = self.layout
        return out
