"""The measurement harness, the tuner and the counter backend on the GPU.

The checks the reference makes of its harness and tuner on a device
(tests/test_benchmark_runner.py:110-149, tests/test_kernels_gpu.py:144-222),
restated for this build:

* the GPU path times with HIP events and flushes before every iteration;
* the flush changes the measurement of a problem whose working set would
  otherwise stay cache-resident -- here a working set that fits the 256 MiB
  Infinity Cache but not L2, the case an L2-only flush would miss;
* the harness agrees with ``torch.utils.benchmark`` within 15%;
* the tuned winner is no slower than the untuned default (5% noise margin);
* a configuration with no instantiation, or one the library refuses at
  launch, becomes a recorded outcome instead of an exception;
* a winner tuned in one process is what a fresh process dispatches;
* ``kernelforge profile --backend rocprof`` returns MFMA utilisation and HBM
  traffic for one launch.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

from kernelforge.benchmark.runner import benchmark, cross_check_median_ms
from kernelforge.tuning.config import KernelConfig, Problem

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
REPO = Path(__file__).resolve().parent.parent


def test_gpu_path_uses_hip_events_and_flushes():
    x = torch.randn(4096, 4096, device=DEV)
    result = benchmark(lambda: x * 2, warmup=5, iterations=20, device=DEV)
    assert result.timer == "hip_event" and result.flushed_l2 is True and result.median_ms > 0
    again = benchmark(lambda: x * 2, warmup=0, iterations=20, device=DEV, flush_l2=False)
    assert again.timer == "hip_event" and not again.flushed_l2


def _medians_after(pre, fn, iterations=100):
    """Median event time of ``fn`` when ``pre`` runs before each start event."""
    start = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
    for _ in range(10):
        fn()
    torch.cuda.synchronize()
    for i in range(iterations):
        pre()
        start[i].record()
        fn()
        end[i].record()
    torch.cuda.synchronize()
    return float(torch.tensor([s.elapsed_time(e) for s, e in zip(start, end)]).median())


def test_flush_evicts_a_working_set_the_infinity_cache_would_hold():
    """A 48 MiB working set (two 16 MiB inputs and a 16 MiB output) is far more
    than the 4 MiB L2 of one XCD and far less than the 256 MiB Infinity Cache.

    Both timings keep the GPU busy before each start event -- the flush in one,
    a spin of about the same length that touches no memory in the other -- so
    the host's launch time is hidden in both and the only difference left is
    where the inputs come from. Without that, an unflushed loop of short
    kernels measures the host's launch rate instead.
    """
    from kernelforge.benchmark.runner import flush_buffer
    from kernelforge.kernels.rmsnorm import rmsnorm
    from kernelforge.kernels.vector_add import vector_add

    flush = flush_buffer(DEV)
    spin = lambda: torch.cuda._sleep(100_000)  # noqa: E731 -- ~50 us at the shader clock
    n = 1 << 22
    a = torch.randn(n, device=DEV)
    b = torch.randn(n, device=DEV)
    add_warm = _medians_after(spin, lambda: vector_add(a, b))
    add_cold = _medians_after(flush.flush, lambda: vector_add(a, b))
    print(f"vector_add 3 x 16 MiB: warm {add_warm * 1e3:.2f} us, cold {add_cold * 1e3:.2f} us",
          flush=True)
    assert add_cold > add_warm * 1.05

    # A row kernel whose 32 MiB working set also fits the Infinity Cache. (A
    # GEMM of this size is MFMA-bound: where its operands come from does not
    # change its time, so it cannot show what the flush does.)
    rows = torch.randn(2048, 2048, device=DEV)
    gamma = torch.ones(2048, device=DEV)
    norm_warm = _medians_after(spin, lambda: rmsnorm(rows, gamma))
    norm_cold = _medians_after(flush.flush, lambda: rmsnorm(rows, gamma))
    print(f"rmsnorm 2048x2048 fp32: warm {norm_warm * 1e3:.2f} us, cold {norm_cold * 1e3:.2f} us",
          flush=True)
    assert norm_cold > norm_warm
    # The harness's own flushed path starts every iteration cold.
    timed = benchmark(lambda: vector_add(a, b), warmup=10, iterations=50, device=DEV)
    assert timed.flushed_l2 and timed.median_ms > add_warm * 1.05


def test_harness_agrees_with_torch_utils_benchmark():
    from kernelforge.kernels.matmul import matmul

    # Long enough (~150 us) that neither timer is bound by the host's launch rate.
    a = torch.randn(4096, 4096, device=DEV, dtype=torch.float16)
    b = torch.randn(4096, 4096, device=DEV, dtype=torch.float16)
    for label, run in (("hipBLASLt", lambda: a @ b), ("kernelforge", lambda: matmul(a, b))):
        ours = benchmark(run, warmup=25, iterations=200, device=DEV, flush_l2=False)
        theirs = cross_check_median_ms(run, min_run_time=0.5)
        print(f"{label}: harness {ours.median_ms * 1e3:.1f} us, torch.utils.benchmark "
              f"{theirs * 1e3:.1f} us")
        assert ours.median_ms == pytest.approx(theirs, rel=0.15)


def test_tuned_winner_is_not_slower_than_the_untuned_default():
    from kernelforge.kernels import get_operator
    from kernelforge.tuning.tuner import Tuner

    result = Tuner(warmup=25, iterations=50, max_candidates=12).tune(
        get_operator("matmul"), Problem.create("matmul", "fp16", M=1024, N=1024, K=1024), device=DEV)
    assert result.best is not None and result.correct > 0
    default = result.baselines["hip_default"]
    print(f"tuned {result.best.median_ms * 1e3:.1f} us ({dict(result.best.config)}), "
          f"default {default.median_ms * 1e3:.1f} us")
    assert result.best.median_ms <= default.median_ms * 1.05


def test_unbuilt_and_refused_configurations_are_recorded_not_raised():
    from kernelforge.kernels import get_operator
    from kernelforge.tuning.tuner import STATUS_COMPILE_ERROR, Tuner, _Trial

    operator = get_operator("matmul")
    problem = Problem.create("matmul", "fp16", M=256, N=256, K=256)
    inputs = operator.make_inputs(problem, DEV)
    reference = operator.reference(*inputs)
    tuner = Tuner()
    missing = _Trial(KernelConfig("matmul", BLOCK_M=48, BLOCK_N=48, BLOCK_K=32, GROUP_M=8,
                                  num_warps=4, num_stages=2))
    tuner._gate(operator, problem, missing, inputs, reference)
    assert missing.status == STATUS_COMPILE_ERROR and "ahead-of-time" in missing.error
    # A GEMV launch shape the library refuses (KF_ERR_OUT_OF_RESOURCES): no launch happens.
    gemv = Problem.create("matmul", "fp16", M=1, N=256, K=256)
    gemv_inputs = operator.make_inputs(gemv, DEV)
    refused = _Trial(KernelConfig("matmul", GEMV=1, SPLIT_K=1, LANES_PER_ROW=16, num_warps=17))
    tuner._gate(operator, gemv, refused, gemv_inputs, operator.reference(*gemv_inputs))
    assert refused.status == STATUS_COMPILE_ERROR and "waves" in refused.error
    assert refused.timing is None


def test_a_winner_tuned_here_is_what_a_fresh_process_dispatches(tmp_path):
    from kernelforge.kernels import get_operator
    from kernelforge.runtime.dispatch import SOURCE_DEFAULT, select_config
    from kernelforge.tuning.cache import ConfigCache
    from kernelforge.tuning.tuner import Tuner

    operator = get_operator("rmsnorm")
    problem = Problem.create("rmsnorm", "fp16", rows=512, cols=1024)
    path = tmp_path / "configs.json"
    fresh = select_config(operator, problem, cache=ConfigCache(path), use_packaged=False)
    assert fresh.source == SOURCE_DEFAULT
    result = Tuner(warmup=5, iterations=20, cache=ConfigCache(path), measure_baselines=False).tune(
        operator, problem, device=DEV)
    assert result.best is not None
    probe = (
        "from kernelforge.kernels import get_operator\n"
        "from kernelforge.runtime.dispatch import select_config\n"
        "from kernelforge.tuning.cache import ConfigCache\n"
        "from kernelforge.tuning.config import Problem\n"
        "p = Problem.create('rmsnorm', 'fp16', rows=512, cols=1024)\n"
        f"s = select_config(get_operator('rmsnorm'), p, cache=ConfigCache({str(path)!r}))\n"
        "print(s.source, s.config.to_json())\n"
    )
    out = subprocess.run([sys.executable, "-c", probe], capture_output=True, text=True, cwd=REPO,
                         timeout=180)
    assert out.returncode == 0, out.stderr
    source, payload = out.stdout.split()
    assert source == "cache"
    assert KernelConfig.from_json("rmsnorm", payload) == result.best_config


@pytest.mark.timeout(600)
@pytest.mark.parametrize("argv,bound", [
    (["matmul", "-m", "2048", "-n", "4096", "-k", "4096", "--dtype", "fp16"], "MFMA"),
    (["rmsnorm", "--rows", "4096", "--cols", "4096", "--dtype", "fp32"], "HBM"),
], ids=("gemm", "rmsnorm"))
def test_profile_rocprof_backend_reads_counters_of_one_launch(argv, bound, tmp_path):
    print(f"profile --backend rocprof {' '.join(argv)}", flush=True)
    out = subprocess.run([sys.executable, "-m", "kernelforge", "profile", *argv, "--backend",
                          "rocprof", "--no-cache", "--profile-dir", str(tmp_path / "prof")],
                         capture_output=True, text=True, cwd=REPO, timeout=560)
    print(out.stdout[-3000:])
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    text = out.stdout
    assert ("kf::" in text or "_ZN2kf" in text) and "duration" in text and "HBM traffic" in text
    assert f"bound: {bound}" in text
    if bound == "MFMA":
        assert "MFMA busy" in text and "MFMA FLOPs" in text
