"""Configuration selection at call time (kernelforge/runtime/dispatch.py:47-64).

    hit  -> the configuration tuning chose for this device and shape
    miss -> the operator's default, with the miss reported

Nothing here tunes: tuning is an explicit step (``tune``) whose output this
reads in microseconds.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

import torch

from kernelforge.kernels.base import Operator
from kernelforge.runtime.env import device_key as resolve_device_key
from kernelforge.tuning.cache import PACKAGED_CACHE, ConfigCache
from kernelforge.tuning.config import KernelConfig, Problem

SOURCE_CACHE = "cache"
SOURCE_PACKAGED = "packaged"
SOURCE_DEFAULT = "default"


@dataclass(frozen=True)
class Selection:
    config: KernelConfig
    source: str
    device_key: str

    @property
    def tuned(self) -> bool:
        return self.source in (SOURCE_CACHE, SOURCE_PACKAGED)

    def describe(self) -> str:
        if self.source == SOURCE_CACHE:
            return f"tuned configuration for {self.device_key}"
        if self.source == SOURCE_PACKAGED:
            return f"packaged tuned configuration for {self.device_key}"
        return f"default configuration (no cache entry for {self.device_key})"


_PACKAGED: ConfigCache | None = None


def packaged_cache() -> ConfigCache | None:
    """The winners shipped with the package (read-only), if present."""
    global _PACKAGED
    if _PACKAGED is None and PACKAGED_CACHE.exists():
        _PACKAGED = ConfigCache(PACKAGED_CACHE, read_only=True)
    return _PACKAGED


def select_config(
    operator: Operator,
    problem: Problem,
    *,
    cache: ConfigCache | None = None,
    device: torch.device | str | None = None,
    use_packaged: bool = True,
) -> Selection:
    """Pick the configuration to run ``problem`` with: the user's cache, then
    the packaged MI355X winners, then the operator default.

    A product over k-contiguous B (``layout="bt"``) looks for winners of its
    own first; without one, MFMA-tile shapes take the row-major winner (both
    layouts run the same tile pipelines at the same speed), decode shapes the
    layout-aware default (their GEMV kernel differs by layout).
    """
    key = resolve_device_key(device)
    resolved = cache if cache is not None else ConfigCache()
    shipped = packaged_cache() if use_packaged else None
    lookups = [problem]
    if problem.layout and problem.dims_dict.get("M", 0) > _GEMV_MAX_M:
        lookups.append(problem.with_layout(""))
    for candidate in lookups:
        cached = resolved.get(candidate, key)
        if cached is not None:
            return Selection(config=cached, source=SOURCE_CACHE, device_key=key)
        if shipped is not None:
            hit = shipped.get(candidate, key)
            if hit is not None:
                return Selection(config=hit, source=SOURCE_PACKAGED, device_key=key)
    return Selection(config=operator.default_config(problem), source=SOURCE_DEFAULT, device_key=key)


#: Rows up to which a product is a decode GEMV (tuning/search.py GEMV_MAX_M).
_GEMV_MAX_M = 8


@lru_cache(maxsize=4096)
def _shipped(operation: str, dtype: torch.dtype, dims: tuple, layout: str,
             device_index: int) -> KernelConfig | None:
    shipped = packaged_cache()
    if shipped is None:
        return None
    problem = Problem.create(operation, dtype, layout=layout, **dict(dims))
    return shipped.get(problem, resolve_device_key(torch.device("cuda", device_index)))


def shipped_config(operation: str, dtype: torch.dtype, device: torch.device, *, layout: str = "",
                   **dims: int) -> KernelConfig | None:
    """The packaged winner for this call's shape on ``device``, if one ships.

    What a kernel entry point runs when the caller passes no configuration
    (the reference runs its fixed ``DEFAULT_CONFIG`` there, matmul.py:118-120):
    the winners are fixed per release, so a shape always gets the same
    configuration, and the lookup is memoised per shape and device so the
    call costs a dictionary probe. The user's own winner cache is consulted
    only through ``select_config``, as in the reference.
    """
    if device.type != "cuda" or min(dims.values()) < 1:
        return None
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _shipped(operation, dtype, tuple(dims.items()), layout, index)
