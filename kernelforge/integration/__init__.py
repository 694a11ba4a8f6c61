"""Consumers of the tuned kernels (kernelforge/integration/__init__.py).

Names resolve lazily so ``import kernelforge.integration`` costs nothing until
the block is used.
"""

from __future__ import annotations

__all__ = ["BACKENDS", "BlockConfig", "TransformerBlock", "benchmark_block"]


def __getattr__(name: str):
    if name in __all__:
        from kernelforge.integration import transformer

        return getattr(transformer, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
