"""Command line interface:
``kernelforge env|tune|benchmark|compare|profile|report|cache``.

Every subcommand is a thin wrapper over a library call (kernelforge/cli/
main.py:23-643):

* ``tune`` over :class:`~kernelforge.tuning.tuner.Tuner`;
* ``benchmark`` runs a named workload suite (``benchmark.workloads``) through
  dispatch, the gate and the timer and records every row in the database;
* ``compare`` times every implementation at one shape, or a whole
  :class:`~kernelforge.integration.TransformerBlock` per backend;
* ``profile`` attributes launches, or makes the single launch that
  ``rocprofv3 --pmc`` wraps for hardware counters;
* ``report`` renders ``summary.md``, CSV and figures from the database;
* ``cache`` lists or clears the winner cache.

Exit codes: 0 success, 1 failure (including no candidate passing the gate),
2 unusable environment; errors print ``error: ...`` to stderr.
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

from kernelforge import __version__
from kernelforge.dtypes import SUPPORTED_DTYPES, parse_dtype
from kernelforge.tuning.config import Problem

_GEMM_OPERATIONS = ("matmul", "fused_linear")
_ROW_OPERATIONS = ("rmsnorm", "softmax")
_DEFAULT_GEMM = {"m": 2048, "n": 4096, "k": 4096}
_DEFAULT_ROW = {"rows": 4096, "cols": 4096}

_DEFAULT_ELEMENTS = 1 << 24

OPERATIONS = (*_GEMM_OPERATIONS, *_ROW_OPERATIONS, "vector_add")


def _rule(title: str) -> str:
    return f"\n{title}\n{'-' * len(title)}"


def build_problem(operation: str, args: argparse.Namespace) -> Problem:
    dtype = parse_dtype(args.dtype)
    if operation in _GEMM_OPERATIONS:
        return Problem.create(
            operation,
            dtype,
            M=args.m or _DEFAULT_GEMM["m"],
            N=args.n or _DEFAULT_GEMM["n"],
            K=args.k or _DEFAULT_GEMM["k"],
        )
    if operation in _ROW_OPERATIONS:
        return Problem.create(
            operation,
            dtype,
            rows=args.rows or _DEFAULT_ROW["rows"],
            cols=args.cols or _DEFAULT_ROW["cols"],
        )
    if operation == "vector_add":
        return Problem.create(operation, dtype, n=args.elements or _DEFAULT_ELEMENTS)
    raise ValueError(f"unknown operation {operation!r}")


def _describe_problem(problem: Problem) -> str:
    from kernelforge.runtime.env import capture_environment

    env = capture_environment()
    shape = " x ".join(str(v) for _, v in problem.dims)
    return "\n".join(
        [
            f"GPU:    {env.gpu_name or 'none (CPU only)'} {env.gpu_arch or ''}".rstrip(),
            f"Shape:  {shape}  ({'/'.join(k for k, _ in problem.dims)})",
            f"dtype:  {problem.dtype_name.upper()}",
        ]
    )


def _open_db(args: argparse.Namespace):
    from kernelforge.db import ResultsDB

    if getattr(args, "no_db", False):
        return None
    return ResultsDB(args.db)


def _open_cache(args: argparse.Namespace):
    from kernelforge.tuning.cache import ConfigCache

    if getattr(args, "no_cache", False):
        return None
    return ConfigCache(args.cache)


# --- env ---------------------------------------------------------------------
def command_env(args: argparse.Namespace) -> int:
    from kernelforge.runtime.env import capture_environment, device_caps

    env = capture_environment()
    print(env.render())
    caps = device_caps()
    if env.gpu_name is None:
        print("\nNo ROCm device: kernels cannot run here; the tuning core still imports.")
        print(f"Search spaces reason over: {caps.name}")
    print(_rule("Device limits"))
    for title, value in (
        ("Compute units", f"{caps.cu_count} in {caps.xcd_count} XCDs"),
        ("LDS per workgroup", f"{caps.lds_per_workgroup / 1024:.0f} KiB"),
        ("Wave size", f"{caps.wave_size}"),
        ("Registers per lane", f"{caps.vgprs_per_lane} VGPR + {caps.agprs_per_lane} AGPR"),
        ("L2 (all XCDs)", f"{caps.l2_cache_bytes / 1024**2:.0f} MiB"),
        ("Infinity Cache", f"{caps.mall_bytes / 1024**2:.0f} MiB"),
        ("Peak fp16/bf16 MFMA", f"{caps.peak_fp16_tflops:.1f} TFLOP/s"),
        ("Peak HBM", f"{caps.peak_hbm_gbps:.0f} GB/s"),
        ("Cache key", caps.key),
    ):
        print(f"{title:<24}{value}")
    return 0


# --- tune ----------------------------------------------------------------------
def _render_tuning(result, operator) -> str:
    from kernelforge.benchmark import metrics

    lines = [_rule("Best configuration")]
    best = result.best
    if best is None:
        lines.append("No configuration passed verification.")
        lines += [f"  {status}: {count}" for status, count in sorted(result.status_counts().items())]
        return "\n".join(lines)
    lines.append(best.config.render(operator.config_order))

    lines.append(_rule("Performance"))
    latencies = sorted(result.baselines.items(), key=lambda kv: kv[1].median_ms)
    latencies.append(("kernelforge", best.timing))
    width = max(len(label) for label, _ in latencies) + 2
    lines += [f"{label + ':':<{width}}{t.median_ms:>9.3f} ms" for label, t in latencies]

    derived = [
        (f"speedup vs {label}", f"{result.speedup_over(label):.2f}x")
        for label in sorted(result.baselines)
        if result.speedup_over(label) is not None
    ]
    if result.memory_bound:
        derived.append(("bandwidth", f"{result.gbps(best.median_ms):.1f} GB/s"))
    else:
        derived.append(("throughput", f"{result.tflops(best.median_ms):.1f} TFLOP/s"))
    derived.append(
        (
            "arithmetic intensity",
            f"{metrics.arithmetic_intensity(result.flops, result.bytes_moved):.1f} FLOP/byte",
        )
    )
    dw = max(len(label) for label, _ in derived) + 2
    lines.append("")
    lines += [f"{label + ':':<{dw}}{value:>16}" for label, value in derived]
    if best.timing is not None and best.timing.at_timer_resolution:
        lines.append(
            "\nWarning: median latency is at event-timer resolution; "
            "use a larger problem for a meaningful comparison."
        )
    return "\n".join(lines)


def command_tune(args: argparse.Namespace) -> int:
    from kernelforge.kernels import get_operator
    from kernelforge.tuning.search import search_space
    from kernelforge.tuning.tuner import Tuner

    problem = build_problem(args.operation, args)
    if args.explain:
        from kernelforge.runtime.env import device_caps

        space = search_space(args.operation)
        if args.max_candidates is not None:
            space.max_candidates = args.max_candidates
        print(space.explain(problem, device_caps()))
        return 0

    operator = get_operator(args.operation)
    print(_describe_problem(problem))
    print()
    db = _open_db(args)
    cache = _open_cache(args)
    try:
        result = Tuner(
            warmup=args.warmup,
            iterations=args.iterations,
            max_candidates=args.max_candidates,
            measure_baselines=not args.no_baselines,
            flush_l2=not args.no_flush_l2,
            db=db,
            cache=cache,
            log=print,
        ).tune(operator, problem)
    finally:
        if db is not None:
            db.close()
    print(
        f"\nSearch space: {result.generated} grid points, {result.feasible} feasible, "
        f"{result.tested} measured in {result.elapsed_s:.1f}s"
    )
    if args.show_all:
        print(_rule("All candidates"))
        for o in sorted(result.outcomes, key=lambda o: (not o.ok, o.timing.median_ms if o.timing else 0)):
            params = " ".join(f"{k}={v}" for k, v in o.config.items())
            if o.timing is not None:
                rate = (
                    f"{result.gbps(o.median_ms):9.1f} GB/s"
                    if result.memory_bound
                    else f"{result.tflops(o.median_ms):9.1f} TFLOP/s"
                )
                print(f"  {o.timing.median_us:9.1f} us {rate}  {params}")
            else:
                print(f"  {o.status:>14}  {params}  {o.error[:120]}")
    print(_render_tuning(result, operator))
    return 0 if result.best is not None else 1


# --- benchmark -----------------------------------------------------------------
def _rate(operator, problem, median_ms: float) -> tuple[str, float | None, float | None]:
    """Headline rate text plus the (tflops, gbps) pair to record."""
    from kernelforge.benchmark import metrics

    if operator.is_memory_bound():
        value = metrics.gbps(operator.bytes_moved(problem), median_ms)
        return f"{value:.1f} GB/s", None, value
    value = metrics.tflops(operator.flops(problem), median_ms)
    return f"{value:.1f} TFLOP/s", value, None


def _cpu_runnable(operator, inputs):
    """torch eager on host copies of the inputs: the ``torch_cpu`` baseline."""
    host = tuple(t.detach().to("cpu") for t in inputs)
    return lambda: operator.reference(*host)


def command_benchmark(args: argparse.Namespace) -> int:
    from kernelforge.benchmark import workloads
    from kernelforge.benchmark.runner import benchmark
    from kernelforge.db import Measurement
    from kernelforge.kernels import get_operator
    from kernelforge.runtime.dispatch import select_config
    from kernelforge.runtime.env import capture_environment, require_gpu
    from kernelforge.testing import exact_fp32_matmul, verify

    device = require_gpu()
    operator = get_operator(args.operation)
    problems = workloads.problems(args.operation, args.suite, args.dtype)
    environment = capture_environment(device)
    cache = _open_cache(args)
    db = _open_db(args)
    run_id = (
        db.start_run(environment, notes=f"benchmark:{args.suite}", version=__version__)
        if db is not None
        else None
    )
    print(environment.render())
    print(_rule(f"{args.operation} / {args.suite} / {args.dtype}"))
    header = f"{'shape':<24}{'impl':<14}{'config':<10}{'median ms':>11}{'p99 ms':>10}{'metric':>16}"
    print(header)
    print("-" * len(header))
    failures = 0
    try:
        for problem in problems:
            inputs = operator.make_inputs(problem, device)
            with exact_fp32_matmul():
                reference = operator.reference(*inputs)
                selection = select_config(operator, problem, cache=cache, device=device)
                runnable = dict(operator.baselines(problem, inputs))
                runnable["kernelforge"] = lambda c=selection.config, i=inputs: operator.run(c, *i)
                if args.cpu_baseline:
                    runnable["torch_cpu"] = _cpu_runnable(operator, inputs)
                for label, fn in runnable.items():
                    source = selection.source if label == "kernelforge" else "-"
                    try:
                        out = fn()
                        check = verify(reference, out.to(reference.device), dtype=problem.dtype)
                    except Exception as exc:  # noqa: BLE001 - reported per row, never fatal
                        failures += label == "kernelforge"
                        print(f"{problem.shape_key:<24}{label:<14}{source:<10}  failed: "
                              f"{type(exc).__name__}: {str(exc)[:80]}")
                        if db is not None:
                            db.record(run_id, problem, Measurement(
                                label=label, status="runtime_error",
                                config=selection.config if label == "kernelforge" else None,
                                error=f"{type(exc).__name__}: {exc}"))
                        continue
                    if not check.passed:
                        failures += label == "kernelforge"
                        print(f"{problem.shape_key:<24}{label:<14}{source:<10}  INCORRECT: "
                              f"{check.reason}")
                        if db is not None:
                            db.record(run_id, problem, Measurement(
                                label=label, status="incorrect", verification=check,
                                config=selection.config if label == "kernelforge" else None))
                        continue
                    on_host = label == "torch_cpu"
                    timing = benchmark(
                        fn,
                        warmup=min(args.warmup, 1) if on_host else args.warmup,
                        iterations=min(args.iterations, 3) if on_host else args.iterations,
                        device="cpu" if on_host else device,
                        flush_l2=not args.no_flush_l2 and not on_host,
                    )
                    text, tflops_value, gbps_value = _rate(operator, problem, timing.median_ms)
                    print(f"{problem.shape_key:<24}{label:<14}{source:<10}"
                          f"{timing.median_ms:>11.4f}{timing.p99_ms:>10.4f}{text:>16}")
                    if db is not None:
                        db.record(run_id, problem, Measurement(
                            label=label, status="ok",
                            config=selection.config if label == "kernelforge" else None,
                            verification=check, timing=timing, tflops=tflops_value,
                            gbps=gbps_value))
    finally:
        if db is not None:
            db.close()
    return 1 if failures else 0


# --- compare -------------------------------------------------------------------
def command_compare(args: argparse.Namespace) -> int:
    if args.operation == "transformer":
        return _compare_transformer(args)

    from kernelforge.benchmark.runner import benchmark
    from kernelforge.kernels import get_operator
    from kernelforge.runtime.dispatch import select_config
    from kernelforge.runtime.env import require_gpu
    from kernelforge.testing import exact_fp32_matmul, verify

    device = require_gpu()
    operator = get_operator(args.operation)
    problem = build_problem(args.operation, args)
    print(_describe_problem(problem))
    inputs = operator.make_inputs(problem, device)
    with exact_fp32_matmul():
        reference = operator.reference(*inputs)
        selection = select_config(operator, problem, cache=_open_cache(args), device=device)
        print(f"config: {selection.describe()}")
        print(f"        {', '.join(f'{k}={v}' for k, v in selection.config.items())}")
        runnable = dict(operator.baselines(problem, inputs))
        runnable["kernelforge"] = lambda: operator.run(selection.config, *inputs)
        print(_rule("Comparison"))
        rows = []
        for label, fn in runnable.items():
            check = verify(reference, fn(), dtype=problem.dtype)
            if not check.passed:
                print(f"{label}: INCORRECT ({check.reason})")
                continue
            timing = benchmark(
                fn, warmup=args.warmup, iterations=args.iterations, device=device,
                flush_l2=not args.no_flush_l2,
            )
            rows.append((label, timing, check))
    rows.sort(key=lambda row: row[1].median_ms)
    eager = next((t.median_ms for label, t, _ in rows if label == "torch_eager"), None)
    header = f"{'impl':<14}{'median ms':>11}{'p99 ms':>10}{'vs eager':>10}{'metric':>16}{'max err':>11}"
    print(header)
    print("-" * len(header))
    for label, timing, check in rows:
        text, _, _ = _rate(operator, problem, timing.median_ms)
        relative = f"{eager / timing.median_ms:.2f}x" if eager else "-"
        print(f"{label:<14}{timing.median_ms:>11.4f}{timing.p99_ms:>10.4f}{relative:>10}"
              f"{text:>16}{check.error:>11.2e}")
    return 0


def _compare_transformer(args: argparse.Namespace) -> int:
    from kernelforge.integration import BlockConfig, benchmark_block
    from kernelforge.runtime.env import require_gpu

    device = require_gpu()
    config = BlockConfig(hidden=args.hidden, heads=args.heads, intermediate=args.intermediate)
    print(
        f"Transformer block: hidden={config.hidden} heads={config.heads} "
        f"intermediate={config.intermediate} batch={args.batch} seq={args.seq} dtype={args.dtype}"
    )
    results = benchmark_block(
        config, batch=args.batch, seq=args.seq, dtype=parse_dtype(args.dtype), device=device,
        warmup=args.warmup, iterations=args.iterations, cache=_open_cache(args),
    )
    print(_rule("Block latency"))
    baseline = results["torch"].median_ms
    for backend, timing in results.items():
        ratio = "" if backend == "torch" else f"  ({baseline / timing.median_ms:.3f}x)"
        print(f"{backend:<14}{timing.median_ms:>10.3f} ms{ratio}")
    print(
        "\nOnly the two RMSNorms and the MLP up-projection with its bias + GELU are swapped;\n"
        "attention and the other projections are PyTorch in both, so the block-level\n"
        "speedup is bounded by the share of block time those operators held."
    )
    return 0


# --- report --------------------------------------------------------------------
def command_report(args: argparse.Namespace) -> int:
    from kernelforge.benchmark import report
    from kernelforge.db import ResultsDB

    path = Path(args.db)
    if not path.exists():
        print(f"no results database at {path}; run `kernelforge tune` first.", file=sys.stderr)
        return 2
    with ResultsDB(path) as db:
        counts = db.counts()
        print(
            f"{counts['results']} measurements across {counts['problems']} problems "
            f"and {counts['runs']} runs"
        )
        print(report.generate(db, args.out).render())
    return 0


# --- profile -------------------------------------------------------------------
def command_profile(args: argparse.Namespace) -> int:
    from kernelforge.kernels import get_operator
    from kernelforge.runtime.dispatch import select_config
    from kernelforge.runtime.env import require_gpu

    device = require_gpu()
    operator = get_operator(args.operation)
    problem = build_problem(args.operation, args)
    inputs = operator.make_inputs(problem, device)
    selection = select_config(operator, problem, cache=_open_cache(args), device=device)

    if args.backend == "launch-once":
        # The target a counter profiler (rocprofv3 --pmc ...) wraps: one launch.
        import torch

        operator.run(selection.config, *inputs)
        torch.cuda.synchronize()
        return 0

    from kernelforge.profiling import compare_launch_counts

    print(_describe_problem(problem))
    print(f"config: {selection.describe()}: {dict(selection.config)}")
    candidates = dict(operator.baselines(problem, inputs))
    candidates["kernelforge"] = lambda: operator.run(selection.config, *inputs)
    print(_rule("Kernel attribution"))
    for result in compare_launch_counts(candidates, warmup=args.warmup, iterations=args.iterations):
        print(result.render())
        print()
    return 0


# --- cache ----------------------------------------------------------------------
def command_cache(args: argparse.Namespace) -> int:
    from kernelforge.tuning.cache import ConfigCache

    cache = ConfigCache(args.cache)
    if args.cache_command == "clear":
        removed = cache.clear()
        print(f"removed {removed} cached configuration(s) from {cache.path}")
        return 0
    entries = cache.entries()
    print(f"{cache.path}: {len(entries)} entry(ies)")
    for entry in entries:
        print(f"  {entry.describe()}")
    return 0


# --- parser ---------------------------------------------------------------------
def _add_shape_arguments(parser: argparse.ArgumentParser) -> None:
    group = parser.add_argument_group("shape", "dimensions; defaults follow the operation")
    group.add_argument("-m", "--m", type=int, help="GEMM rows of A (matmul, fused_linear)")
    group.add_argument("-n", "--n", type=int, help="GEMM columns of B (matmul, fused_linear)")
    group.add_argument("-k", "--k", type=int, help="GEMM reduction size (matmul, fused_linear)")
    group.add_argument("--rows", type=int, help="rows (rmsnorm, softmax)")
    group.add_argument("--cols", type=int, help="row width (rmsnorm, softmax)")
    group.add_argument("--elements", type=int, help="element count (vector_add)")


def _add_measurement_arguments(parser: argparse.ArgumentParser, *, warmup=25, iterations=200):
    parser.add_argument("--dtype", default="fp16", choices=SUPPORTED_DTYPES)
    parser.add_argument("--warmup", type=int, default=warmup)
    parser.add_argument("--iterations", type=int, default=iterations)
    parser.add_argument(
        "--no-flush-l2",
        action="store_true",
        help="do not flush L2 + Infinity Cache between iterations (inflates cache-resident problems)",
    )


def _add_storage_arguments(parser: argparse.ArgumentParser) -> None:
    from kernelforge.db import default_db_path
    from kernelforge.tuning.cache import default_cache_path

    parser.add_argument("--db", default=str(default_db_path()), help="results database path")
    parser.add_argument("--no-db", action="store_true", help="do not record results")
    parser.add_argument("--cache", default=str(default_cache_path()), help="config cache path")
    parser.add_argument("--no-cache", action="store_true", help="ignore and do not write the cache")


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(
        prog="kernelforge",
        description="Hardware-aware kernel autotuning on MI355X (gfx950).",
    )
    parser.add_argument("--version", action="version", version=f"kernelforge {__version__}")
    sub = parser.add_subparsers(dest="command", required=True)

    sub.add_parser("env", help="print GPU, driver and library versions and device limits")

    tune = sub.add_parser("tune", help="search configurations for one problem")
    tune.add_argument("operation", choices=OPERATIONS)
    _add_shape_arguments(tune)
    _add_measurement_arguments(tune)
    _add_storage_arguments(tune)
    tune.add_argument("--max-candidates", type=int, help="override the candidate budget")
    tune.add_argument("--no-baselines", action="store_true", help="skip comparison baselines")
    tune.add_argument("--show-all", action="store_true", help="print every candidate's outcome")
    tune.add_argument(
        "--explain",
        action="store_true",
        help="print the candidate-generation breakdown and exit without tuning",
    )

    bench = sub.add_parser("benchmark", help="run a named workload suite")
    bench.add_argument("operation", choices=OPERATIONS)
    bench.add_argument("--suite", default="sweep", choices=("smoke", "sweep", "transformer"))
    _add_measurement_arguments(bench, iterations=100)
    _add_storage_arguments(bench)
    bench.add_argument(
        "--cpu-baseline",
        action="store_true",
        help="also time torch eager on the host cores (label torch_cpu; 3 iterations)",
    )

    compare = sub.add_parser(
        "compare", help="compare implementations at one shape, or a whole transformer block"
    )
    compare.add_argument("operation", choices=(*OPERATIONS, "transformer"))
    _add_shape_arguments(compare)
    _add_measurement_arguments(compare, iterations=100)
    _add_storage_arguments(compare)
    compare.add_argument("--batch", type=int, default=1, help="transformer: batch size")
    compare.add_argument("--seq", type=int, default=2048, help="transformer: sequence length")
    compare.add_argument("--hidden", type=int, default=4096, help="transformer: hidden size")
    compare.add_argument("--heads", type=int, default=32, help="transformer: attention heads")
    compare.add_argument(
        "--intermediate", type=int, default=11008, help="transformer: MLP intermediate size"
    )

    profile = sub.add_parser("profile", help="attribute device time and launches to kernels")
    profile.add_argument("operation", choices=OPERATIONS)
    _add_shape_arguments(profile)
    _add_measurement_arguments(profile, warmup=10, iterations=20)
    _add_storage_arguments(profile)
    profile.add_argument(
        "--backend",
        default="torch",
        choices=("torch", "launch-once"),
        help="torch: kernel attribution via torch.profiler; launch-once: a single launch, "
        "the target for `rocprofv3 --pmc ... -- kernelforge profile ... --backend launch-once`",
    )

    report = sub.add_parser("report", help="render tables and figures from the database")
    _add_storage_arguments(report)
    report.add_argument("--out", default="reports", help="output directory")

    cache = sub.add_parser("cache", help="inspect or clear the tuned-config cache")
    cache.add_argument("cache_command", choices=("list", "clear"))
    _add_storage_arguments(cache)
    return parser


_COMMANDS = {
    "env": command_env,
    "tune": command_tune,
    "benchmark": command_benchmark,
    "compare": command_compare,
    "profile": command_profile,
    "report": command_report,
    "cache": command_cache,
}


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    try:
        return _COMMANDS[args.command](args)
    except KeyboardInterrupt:
        print("\ninterrupted", file=sys.stderr)
        return 130
    except (RuntimeError, ValueError) as exc:
        print(f"error: {exc}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    raise SystemExit(main())
