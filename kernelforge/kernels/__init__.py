"""Kernel registry and the public kernel entry points.

Operators resolve lazily by name (kernelforge/kernels/__init__.py:17-38), so
``import kernelforge.kernels`` never loads ``libkernelforge_hip.so`` or creates a
HIP context; the library loads on the first kernel call.
"""

from __future__ import annotations

import importlib
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    from kernelforge.kernels.base import Operator

_OPERATORS: dict[str, tuple[str, str]] = {
    "vector_add": ("kernelforge.kernels.vector_add", "VectorAddOperator"),
    "softmax": ("kernelforge.kernels.softmax", "SoftmaxOperator"),
    "matmul": ("kernelforge.kernels.matmul", "MatmulOperator"),
    "rmsnorm": ("kernelforge.kernels.rmsnorm", "RMSNormOperator"),
    "fused_linear": ("kernelforge.kernels.fused_linear", "FusedLinearOperator"),
}

_FUNCTIONS: dict[str, str] = {
    "vector_add": "kernelforge.kernels.vector_add",
    "matmul": "kernelforge.kernels.matmul",
    "fused_linear_gelu": "kernelforge.kernels.fused_linear",
    "softmax": "kernelforge.kernels.softmax",
    "rmsnorm": "kernelforge.kernels.rmsnorm",
}


def operator_names() -> tuple[str, ...]:
    return tuple(_OPERATORS)


def get_operator(name: str) -> Operator:
    try:
        module_path, class_name = _OPERATORS[name]
    except KeyError:
        raise ValueError(
            f"unknown operator {name!r}; available: {', '.join(operator_names())}"
        ) from None
    module = importlib.import_module(module_path)
    return getattr(module, class_name)()


def __getattr__(name: str) -> Any:
    if name in _FUNCTIONS:
        return getattr(importlib.import_module(_FUNCTIONS[name]), name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
