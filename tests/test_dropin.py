"""The drop-in surface: the reference's import paths and console script, unchanged.

A KernelForge caller imports from ``kernelforge.*`` and runs ``kernelforge
<verb>`` (the reference's pyproject.toml:33-34 maps the script to
``kernelforge.cli.main:main``). Every public name on the hot path must resolve
at the same path with the same call signature, without touching a GPU.
"""

from __future__ import annotations

import importlib
import inspect
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent

#: (module, name, parameters in order) -- the reference's signatures
#: (kernels/matmul.py:132, fused_linear.py:112, softmax.py:70, rmsnorm.py:81).
SURFACE = [
    ("kernelforge.kernels.matmul", "matmul", ["a", "b", "config"]),
    ("kernelforge.kernels.fused_linear", "fused_linear_gelu", ["x", "w", "bias", "config"]),
    ("kernelforge.kernels.softmax", "softmax", ["x", "config"]),
    ("kernelforge.kernels.rmsnorm", "rmsnorm", ["x", "gamma", "eps", "config"]),
    ("kernelforge.kernels.vector_add", "vector_add", ["a", "b", "config"]),
    ("kernelforge.kernels", "get_operator", ["name"]),
    ("kernelforge.kernels.base", "Operator", None),
    ("kernelforge.tuning.config", "KernelConfig", None),
    ("kernelforge.tuning.config", "Problem", None),
    ("kernelforge.tuning.tuner", "Tuner", None),
    ("kernelforge.tuning.cache", "ConfigCache", None),
    ("kernelforge.tuning.search", "SearchSpace", None),
    ("kernelforge.testing", "verify", ["reference", "output", "dtype", "threshold"]),
    ("kernelforge.testing", "assert_verified", None),
    ("kernelforge.testing", "exact_fp32_matmul", None),
    ("kernelforge.db", "ResultsDB", None),
    ("kernelforge.db", "Measurement", None),
    ("kernelforge.runtime.dispatch", "select_config", ["operator", "problem", "cache", "device",
                                                       "use_packaged"]),
    ("kernelforge.runtime.env", "device_caps", None),
    ("kernelforge.benchmark.runner", "benchmark", None),
    ("kernelforge.benchmark.runner", "summarize", None),
    ("kernelforge.benchmark.workloads", "problems", None),
    ("kernelforge.benchmark.report", "generate", None),
    ("kernelforge.integration", "TransformerBlock", None),
    ("kernelforge.integration", "BlockConfig", None),
    ("kernelforge.integration", "benchmark_block", None),
    ("kernelforge.integration.transformer", "BACKEND_KERNELFORGE", None),
    ("kernelforge.integration.transformer", "BACKEND_TORCH", None),
    ("kernelforge.integration.transformer", "BACKENDS", None),
    ("kernelforge.profiling", "profile_kernels", None),
    ("kernelforge.cli.main", "main", ["argv"]),
]


@pytest.mark.parametrize("module,name,params", SURFACE, ids=[f"{m}.{n}" for m, n, _ in SURFACE])
def test_reference_names_resolve_at_their_paths(module, name, params):
    obj = getattr(importlib.import_module(module), name)
    if params is not None:
        assert list(inspect.signature(obj).parameters) == params


def test_the_console_script_is_declared_and_runs():
    import tomli

    project = tomli.loads((REPO / "pyproject.toml").read_text())["project"]
    assert project["name"] == "kernelforge"
    target = project["scripts"]["kernelforge"]
    assert target == "kernelforge.cli.main:main"
    module, func = target.split(":")
    # What the installed script does: import the target and call it with argv.
    script = f"import sys; from {module} import {func}; sys.exit({func}())"
    out = subprocess.run([sys.executable, "-c", script, "tune", "matmul", "--m", "2048", "--n",
                          "4096", "--k", "4096", "--dtype", "fp16", "--explain"],
                         capture_output=True, text=True, cwd=REPO, timeout=300)
    assert out.returncode == 0, out.stderr
    assert "grid points" in out.stdout and "selected (budget)" in out.stdout
