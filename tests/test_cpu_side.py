"""CPU-side behaviour: import hygiene, wrapper validation, CLI, timing statistics.

* Importing the package and every CPU module loads no HIP library and creates
  no GPU context (reference tests/test_cpu_only_imports.py:22-84).
* Kernel wrappers validate shapes, dtypes and layouts before any device touch
  and raise the reference's messages (tests/test_kernel_validation.py).
* The CLI parses, reports the environment, explains a search space and
  manages the cache without a GPU (tests/test_cli.py:20-186).
* ``summarize`` agrees with numpy and the CPU timer labels itself
  (tests/test_benchmark_runner.py:24-107).
"""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

REPO = Path(__file__).resolve().parent.parent

# --- import hygiene -------------------------------------------------------------------

_MODULES = [
    "kernelforge",
    "kernelforge.dtypes",
    "kernelforge.testing",
    "kernelforge.db",
    "kernelforge.tuning.config",
    "kernelforge.tuning.search",
    "kernelforge.tuning.cache",
    "kernelforge.tuning.tuner",
    "kernelforge.runtime.env",
    "kernelforge.runtime.dispatch",
    "kernelforge.runtime.hip",
    "kernelforge.kernels",
    "kernelforge.kernels.matmul",
    "kernelforge.kernels.fused_linear",
    "kernelforge.kernels.softmax",
    "kernelforge.kernels.rmsnorm",
    "kernelforge.benchmark.runner",
    "kernelforge.benchmark.metrics",
    "kernelforge.benchmark.workloads",
    "kernelforge.profiling",
    "kernelforge.cli.main",
]


def test_imports_load_no_hip_library_and_no_context():
    code = f"""
import sys, json
sys.path.insert(0, {str(REPO)!r})
mods = {_MODULES!r}
for m in mods:
    __import__(m)
from kernelforge.runtime import hip
loaded = [l for l in open('/proc/self/maps') if 'libkernelforge_hip' in l]
import torch
print(json.dumps({{"lib_loaded": hip.is_loaded(), "mapped": len(loaded),
                   "cuda_initialized": torch.cuda.is_initialized()}}))
"""
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    state = json.loads(out.stdout.strip().splitlines()[-1])
    assert state == {"lib_loaded": False, "mapped": 0, "cuda_initialized": False}


# --- wrapper validation (CPU tensors, before any device touch) -----------------------


def test_matmul_validation_messages():
    from kernelforge.kernels.matmul import matmul

    with pytest.raises(ValueError, match="2D"):
        matmul(torch.ones(2, 2, 2), torch.ones(2, 2))
    with pytest.raises(ValueError, match="shape mismatch"):
        matmul(torch.ones(2, 3), torch.ones(2, 3))
    with pytest.raises(ValueError, match="dtype mismatch"):
        matmul(torch.ones(2, 2), torch.ones(2, 2, dtype=torch.float16))
    with pytest.raises(ValueError, match="ROCm device tensor"):
        matmul(torch.ones(2, 2), torch.ones(2, 2))


def test_fused_linear_validation_messages():
    from kernelforge.kernels.fused_linear import fused_linear_gelu

    x, w = torch.ones(2, 3), torch.ones(3, 4)
    with pytest.raises(ValueError, match="2D"):
        fused_linear_gelu(torch.ones(3), w, torch.ones(4))
    with pytest.raises(ValueError, match="shape mismatch"):
        fused_linear_gelu(x, torch.ones(2, 4), torch.ones(4))
    with pytest.raises(ValueError, match="bias must have shape"):
        fused_linear_gelu(x, w, torch.ones(3))
    with pytest.raises(ValueError, match="dtype mismatch"):
        fused_linear_gelu(x, w, torch.ones(4, dtype=torch.float16))


def test_row_kernel_validation_messages():
    from kernelforge.kernels.rmsnorm import rmsnorm
    from kernelforge.kernels.softmax import softmax
    from kernelforge.tuning.config import KernelConfig

    with pytest.raises(ValueError, match="2D"):
        softmax(torch.ones(3))
    with pytest.raises(ValueError, match="contiguous last dimension"):
        softmax(torch.ones(4, 4).t())
    with pytest.raises(ValueError, match="cannot hold a row"):
        softmax(torch.ones(4, 300), config=KernelConfig("softmax", BLOCK_SIZE=256, ROWS_PER_PROGRAM=1,
                                                        num_warps=1))
    with pytest.raises(ValueError, match="single-pass limit"):
        softmax(torch.ones(2, 16385))
    with pytest.raises(ValueError, match="gamma must have shape"):
        rmsnorm(torch.ones(2, 8), torch.ones(7))
    with pytest.raises(ValueError, match="gamma must be contiguous"):
        rmsnorm(torch.ones(2, 8), torch.ones(8, 2)[:, 0])
    single_pass = KernelConfig("rmsnorm", BLOCK_SIZE=32768, ROWS_PER_PROGRAM=1, num_warps=16)
    with pytest.raises(ValueError, match="single-pass limit"):
        rmsnorm(torch.ones(2, 16385), torch.ones(16385), config=single_pass)
    # Without a config, a row past the limit takes the two-pass kernel, which
    # still refuses host tensors before anything reaches the library.
    with pytest.raises(ValueError, match="ROCm device tensor"):
        rmsnorm(torch.ones(2, 16385), torch.ones(16385))
    with pytest.raises(ValueError, match="ROCm device tensor"):
        rmsnorm(torch.ones(2, 8), torch.ones(8))


def test_vector_add_validation_messages():
    from kernelforge.kernels.vector_add import vector_add

    a = torch.zeros(8, dtype=torch.float16)
    with pytest.raises(ValueError, match="shape mismatch"):
        vector_add(a, torch.zeros(9, dtype=torch.float16))
    with pytest.raises(ValueError, match="dtype mismatch"):
        vector_add(a, torch.zeros(8, dtype=torch.float32))
    with pytest.raises(ValueError, match="ROCm device tensor"):
        vector_add(a, a)


def test_registry_is_lazy_and_named():
    from kernelforge.kernels import get_operator, operator_names

    assert set(operator_names()) == {"vector_add", "softmax", "matmul", "rmsnorm", "fused_linear"}
    assert get_operator("rmsnorm").name == "rmsnorm"
    assert get_operator("vector_add").is_memory_bound()
    with pytest.raises(ValueError, match="unknown operator"):
        get_operator("layernorm")


def test_operators_draw_inputs_on_the_cpu_reproducibly():
    from kernelforge.kernels import get_operator
    from kernelforge.tuning.config import Problem

    op = get_operator("fused_linear")
    p = Problem.create("fused_linear", "fp16", M=4, N=8, K=16)
    a = op.make_inputs(p, torch.device("cpu"), seed=3)
    b = op.make_inputs(p, torch.device("cpu"), seed=3)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    assert [t.shape for t in a] == [(4, 16), (16, 8), (8,)]
    assert op.flops(p) == 2 * 4 * 8 * 16
    assert op.bytes_moved(p) == (4 * 16 + 16 * 8 + 8 + 4 * 8) * 2


# --- CLI ---------------------------------------------------------------------------


def _cli(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, "-m", "kernelforge", *args], capture_output=True,
                          text=True, cwd=REPO, timeout=300)


def test_cli_explain_and_env_work_without_a_gpu():
    out = _cli("tune", "matmul", "--m", "2048", "--n", "4096", "--k", "4096", "--explain")
    assert out.returncode == 0, out.stderr
    assert "grid points      : 640" in out.stdout and "no device attached" in out.stdout
    out = _cli("env")
    assert out.returncode == 0 and "Device limits" in out.stdout and "gfx950" in out.stdout


def test_cli_cache_list_and_clear(tmp_path):
    from kernelforge.tuning.cache import ConfigCache
    from kernelforge.tuning.config import KernelConfig, Problem

    path = tmp_path / "c.json"
    ConfigCache(path).put(Problem.create("matmul", "fp16", M=1, N=2, K=3), "dev", KernelConfig("matmul", A=1))
    out = _cli("cache", "list", "--cache", str(path))
    assert out.returncode == 0 and "1 entry" in out.stdout and "1x2x3" in out.stdout
    out = _cli("cache", "clear", "--cache", str(path))
    assert out.returncode == 0 and "removed 1" in out.stdout and not path.exists()


def test_cli_errors_exit_nonzero_with_message():
    out = _cli("tune", "matmul", "--dtype", "fp16", "--m=-5", "--explain")
    assert out.returncode == 1 and out.stderr.startswith("error:")
    out = _cli("tune", "nope")
    assert out.returncode == 2


def test_cli_parser_defaults():
    from kernelforge.cli.main import build_parser, build_problem

    args = build_parser().parse_args(["tune", "rmsnorm"])
    p = build_problem("rmsnorm", args)
    assert p.dims_dict == {"rows": 4096, "cols": 4096} and p.dtype_name == "fp16"
    args = build_parser().parse_args(["tune", "vector_add", "--elements", "1000003"])
    assert build_problem("vector_add", args).dims_dict == {"n": 1000003}
    args = build_parser().parse_args(["benchmark", "softmax", "--suite", "smoke"])
    assert (args.suite, args.iterations, args.cpu_baseline) == ("smoke", 100, False)
    args = build_parser().parse_args(["compare", "transformer", "--seq", "7"])
    assert (args.batch, args.seq, args.hidden, args.heads, args.intermediate) == (1, 7, 4096, 32, 11008)
    args = build_parser().parse_args(["report", "--db", "x.db", "--out", "r"])
    assert (args.db, args.out) == ("x.db", "r")


def test_cli_commands_that_need_a_gpu_say_so():
    for argv in (["benchmark", "vector_add", "--suite", "smoke", "--no-db"],
                 ["compare", "rmsnorm", "--rows", "8", "--cols", "8"],
                 ["compare", "transformer", "--seq", "1"]):
        out = _cli(*argv)
        assert out.returncode == 1 and "require a ROCm GPU" in out.stderr, argv


def test_cli_report_without_a_database_exits_2(tmp_path):
    out = _cli("report", "--db", str(tmp_path / "none.db"), "--out", str(tmp_path / "r"))
    assert out.returncode == 2 and "no results database" in out.stderr


# --- timing statistics -----------------------------------------------------------------


def test_summarize_agrees_with_numpy():
    from kernelforge.benchmark.runner import summarize

    samples = np.random.default_rng(0).gamma(2.0, 0.01, 200)
    r = summarize(samples, warmup=3, iterations=200, timer="hip_event", flushed_l2=True, keep_samples=True)
    assert r.median_ms == pytest.approx(np.median(samples))
    assert r.mean_ms == pytest.approx(samples.mean())
    assert r.std_ms == pytest.approx(samples.std(ddof=1))
    assert r.p95_ms == pytest.approx(np.percentile(samples, 95))
    assert r.p99_ms == pytest.approx(np.percentile(samples, 99))
    assert len(r.samples_ms) == 200 and r.as_dict()["timer"] == "hip_event"
    with pytest.raises(ValueError):
        summarize([], warmup=0, iterations=0, timer="x", flushed_l2=False)


def test_median_is_robust_to_an_outlier():
    from kernelforge.benchmark.runner import summarize

    r = summarize([1.0] * 99 + [1000.0], warmup=0, iterations=100, timer="x", flushed_l2=False)
    assert r.median_ms == 1.0 and r.max_ms == 1000.0


def test_cpu_timing_is_labelled_perf_counter():
    from kernelforge.benchmark.runner import benchmark

    r = benchmark(lambda: sum(range(100)), warmup=1, iterations=5, device="cpu")
    assert r.timer == "perf_counter" and not r.flushed_l2 and r.iterations == 5
    with pytest.raises(ValueError):
        benchmark(lambda: None, iterations=0, device="cpu")


def test_metrics():
    from kernelforge.benchmark import metrics

    assert metrics.matmul_flops(2048, 4096, 4096) == 68719476736
    assert metrics.rmsnorm_bytes(4096, 4096, 4) == 134234112
    assert metrics.softmax_bytes(8192, 11008, 2) == 360710144
    assert metrics.matmul_bytes(1, 11008, 4096, 2) == 90207744
    assert metrics.fused_linear_bytes(4096, 11008, 4096, 2, fused=True) == 213931520
    assert metrics.fused_linear_bytes(4096, 11008, 4096, 2, fused=False) == 574641664
    assert metrics.arithmetic_intensity(68719476736, 67108864) == pytest.approx(1024.0)
    assert metrics.tflops(10**12, 1000.0) == pytest.approx(1.0)
    with pytest.raises(ValueError):
        metrics.gbps(1, 0.0)
