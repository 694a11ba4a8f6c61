"""``kernelforge env|tune|benchmark|compare|profile|report|cache``.

The verbs, flags, exit codes and messages are the reference's
(kernelforge/cli/main.py:23-643), so scripts written against it keep working:
exit 0 on success, 1 on failure (including "no candidate passed the gate"),
2 when the environment cannot do what was asked, and ``error: ...`` on
stderr.

How it is put together here:

* every subcommand is a :class:`_Command` in one registry: it adds its own
  arguments and runs against a :class:`_Session`;
* the session opens what a command touches, lazily and once -- the GPU, the
  results database, the winner cache, the run record -- and closes it all on
  the way out, so no command manages its own handles;
* ``benchmark`` and ``compare`` share one routine (:func:`_evaluate`) that
  gates every implementation against the reference before timing it;
* ``profile --backend rocprof`` re-runs this CLI as a one-launch child under
  ``rocprofv3`` for MFMA utilisation and HBM traffic
  (:mod:`kernelforge.profiling.rocprof`); the parent never touches the GPU.
"""

from __future__ import annotations

import argparse
import sys
import tempfile
from collections.abc import Callable
from dataclasses import dataclass
from pathlib import Path

from kernelforge import __version__
from kernelforge.dtypes import SUPPORTED_DTYPES, parse_dtype
from kernelforge.tuning.config import Problem

#: Operations and the dimensions their problems are built from, with defaults.
_SHAPES: dict[str, tuple[tuple[str, str, int], ...]] = {
    "matmul": (("M", "m", 2048), ("N", "n", 4096), ("K", "k", 4096)),
    "fused_linear": (("M", "m", 2048), ("N", "n", 4096), ("K", "k", 4096)),
    "rmsnorm": (("rows", "rows", 4096), ("cols", "cols", 4096)),
    "softmax": (("rows", "rows", 4096), ("cols", "cols", 4096)),
    "vector_add": (("n", "elements", 1 << 24),),
}
OPERATIONS = tuple(_SHAPES)
TUNED_LABEL = "kernelforge"


def build_problem(operation: str, args: argparse.Namespace) -> Problem:
    """The problem the shape flags describe; unset flags take the operation's defaults."""
    if operation not in _SHAPES:
        raise ValueError(f"unknown operation {operation!r}")
    dims = {dim: getattr(args, flag, None) or default for dim, flag, default in _SHAPES[operation]}
    layout = "bt" if getattr(args, "b_layout", "kn") == "nk" else ""
    if layout and operation not in ("matmul", "fused_linear"):
        raise ValueError(f"--b-layout applies to matmul and fused_linear, not {operation}")
    return Problem.create(operation, parse_dtype(args.dtype), layout=layout, **dims)


def _heading(title: str) -> str:
    return f"\n{title}\n{'-' * len(title)}"


class _Table:
    """Column-aligned rows printed as they arrive."""

    def __init__(self, columns: list[tuple[str, int]]) -> None:
        self.columns = columns  # (title, width); a negative width left-aligns

    def _fmt(self, cells) -> str:
        return "".join(f"{str(c):<{-w}}" if w < 0 else f"{str(c):>{w}}"
                       for c, (_, w) in zip(cells, self.columns))

    def header(self) -> None:
        line = self._fmt([t for t, _ in self.columns])
        print(line)
        print("-" * len(line))

    def row(self, *cells) -> None:
        print(self._fmt(cells))


class _Session:
    """What one invocation opens: device, database, cache, run id. Closed on exit."""

    def __init__(self, args: argparse.Namespace) -> None:
        self.args = args
        self._device = None
        self._db = None
        self._db_opened = False
        self._cache = None
        self._cache_opened = False
        self._run_ids: dict[str, int] = {}

    def __enter__(self) -> _Session:
        return self

    def __exit__(self, *exc: object) -> None:
        if self._db is not None:
            self._db.close()

    @property
    def device(self):
        if self._device is None:
            from kernelforge.runtime.env import require_gpu

            self._device = require_gpu()
        return self._device

    @property
    def db(self):
        if not self._db_opened:
            self._db_opened = True
            if not getattr(self.args, "no_db", False):
                from kernelforge.db import ResultsDB

                self._db = ResultsDB(self.args.db)
        return self._db

    @property
    def cache(self):
        if not self._cache_opened:
            self._cache_opened = True
            if not getattr(self.args, "no_cache", False):
                from kernelforge.tuning.cache import ConfigCache

                self._cache = ConfigCache(self.args.cache)
        return self._cache

    def run_id(self, notes: str) -> int | None:
        if self.db is None:
            return None
        if notes not in self._run_ids:
            from kernelforge.runtime.env import capture_environment

            self._run_ids[notes] = self.db.start_run(capture_environment(self.device), notes=notes,
                                                     version=__version__)
        return self._run_ids[notes]

    def record(self, notes: str, problem: Problem, measurement) -> None:
        run = self.run_id(notes)
        if run is not None:
            self.db.record(run, problem, measurement)

    def select(self, operator, problem: Problem):
        from kernelforge.runtime.dispatch import select_config

        return select_config(operator, problem, cache=self.cache, device=self.device)


@dataclass
class _Command:
    name: str
    help: str
    configure: Callable[[argparse.ArgumentParser], None]
    run: Callable[[_Session], int]


_REGISTRY: dict[str, _Command] = {}


def _command(name: str, help: str, configure: Callable[[argparse.ArgumentParser], None]):
    def register(run: Callable[[_Session], int]) -> Callable[[_Session], int]:
        _REGISTRY[name] = _Command(name, help, configure, run)
        return run

    return register


# --- shared argument groups --------------------------------------------------------------
def _shape_arguments(p: argparse.ArgumentParser) -> None:
    g = p.add_argument_group("shape", "dimensions; unset ones take the operation's defaults")
    g.add_argument("-m", "--m", type=int, help="GEMM rows of A (matmul, fused_linear)")
    g.add_argument("-n", "--n", type=int, help="GEMM columns of B (matmul, fused_linear)")
    g.add_argument("-k", "--k", type=int, help="GEMM reduction size (matmul, fused_linear)")
    g.add_argument("--rows", type=int, help="rows (rmsnorm, softmax)")
    g.add_argument("--cols", type=int, help="row width (rmsnorm, softmax)")
    g.add_argument("--elements", type=int, help="element count (vector_add)")
    g.add_argument("--b-layout", choices=("kn", "nk"), default="kn",
                   help="how B is stored: kn = (K, N) row-major (default); nk = an nn.Linear "
                        "weight (N, K), passed as weight.t() (matmul, fused_linear)")


def _timing_arguments(p: argparse.ArgumentParser, warmup: int = 25, iterations: int = 200) -> None:
    p.add_argument("--dtype", default="fp16", choices=SUPPORTED_DTYPES)
    p.add_argument("--warmup", type=int, default=warmup)
    p.add_argument("--iterations", type=int, default=iterations)
    p.add_argument("--no-flush-l2", action="store_true",
                   help="do not flush L2 + Infinity Cache before each iteration "
                        "(inflates cache-resident problems)")


def _storage_arguments(p: argparse.ArgumentParser) -> None:
    from kernelforge.db import default_db_path
    from kernelforge.tuning.cache import default_cache_path

    p.add_argument("--db", default=str(default_db_path()), help="results database path")
    p.add_argument("--no-db", action="store_true", help="do not record results")
    p.add_argument("--cache", default=str(default_cache_path()), help="winner cache path")
    p.add_argument("--no-cache", action="store_true", help="neither read nor write the cache")


def _operation_arguments(choices=OPERATIONS) -> Callable[[argparse.ArgumentParser], None]:
    def add(p: argparse.ArgumentParser) -> None:
        p.add_argument("operation", choices=choices)
        _shape_arguments(p)

    return add


def _compose(*parts: Callable[[argparse.ArgumentParser], None]):
    def add(p: argparse.ArgumentParser) -> None:
        for part in parts:
            part(p)

    return add


def _problem_banner(problem: Problem) -> str:
    from kernelforge.runtime.env import capture_environment

    env = capture_environment()
    names = "/".join(k for k, _ in problem.dims)
    shape = " x ".join(str(v) for _, v in problem.dims)
    gpu = f"{env.gpu_name or 'none (CPU only)'} {env.gpu_arch or ''}".rstrip()
    return f"GPU:    {gpu}\nShape:  {shape}  ({names})\ndtype:  {problem.dtype_name.upper()}"


def _rate(operator, problem: Problem, median_ms: float) -> tuple[str, float | None, float | None]:
    """Headline text plus the (tflops, gbps) pair to record for one latency."""
    from kernelforge.benchmark import metrics

    if operator.is_memory_bound():
        gbps = metrics.gbps(operator.bytes_moved(problem), median_ms)
        return f"{gbps:.1f} GB/s", None, gbps
    tflops = metrics.tflops(operator.flops(problem), median_ms)
    return f"{tflops:.1f} TFLOP/s", tflops, None


# --- env ---------------------------------------------------------------------------------
@_command("env", "print GPU, driver and library versions and device limits", lambda p: None)
def _env(session: _Session) -> int:
    from kernelforge.runtime.env import capture_environment, device_caps

    env = capture_environment()
    caps = device_caps()
    print(env.render())
    if env.gpu_name is None:
        print("\nNo ROCm device: kernels cannot run here; the tuning core still imports.")
        print(f"Search spaces reason over: {caps.name}")
    print(_heading("Device limits"))
    for title, value in (
        ("Compute units", f"{caps.cu_count} in {caps.xcd_count} XCDs"),
        ("LDS per workgroup", f"{caps.lds_per_workgroup // 1024} KiB"),
        ("Wave size", str(caps.wave_size)),
        ("Registers per lane", f"{caps.vgprs_per_lane} VGPR + {caps.agprs_per_lane} AGPR"),
        ("L2 (all XCDs)", f"{caps.l2_cache_bytes / 2**20:.0f} MiB"),
        ("Infinity Cache", f"{caps.mall_bytes / 2**20:.0f} MiB"),
        ("Peak fp16/bf16 MFMA", f"{caps.peak_fp16_tflops:.1f} TFLOP/s"),
        ("Peak HBM", f"{caps.peak_hbm_gbps:.0f} GB/s"),
        ("Cache key", caps.key),
    ):
        print(f"{title:<24}{value}")
    return 0


# --- tune --------------------------------------------------------------------------------
def _tune_arguments(p: argparse.ArgumentParser) -> None:
    p.add_argument("--max-candidates", type=int, help="override the candidate budget")
    p.add_argument("--no-baselines", action="store_true", help="skip comparison baselines")
    p.add_argument("--show-all", action="store_true", help="print every candidate's outcome")
    p.add_argument("--explain", action="store_true",
                   help="print the candidate-generation breakdown and exit without tuning")


def _tuning_summary(result, operator) -> str:
    from kernelforge.benchmark import metrics

    best = result.best
    out = [_heading("Best configuration")]
    if best is None:
        out.append("No configuration passed verification.")
        out += [f"  {s}: {n}" for s, n in sorted(result.status_counts().items())]
        return "\n".join(out)
    out.append(best.config.render(operator.config_order))
    out.append(_heading("Performance"))
    times = sorted(result.baselines.items(), key=lambda kv: kv[1].median_ms)
    times.append((TUNED_LABEL, best.timing))
    w = 2 + max(len(label) for label, _ in times)
    out += [f"{(label + ':').ljust(w)}{t.median_ms:>9.3f} ms" for label, t in times]
    facts = [(f"speedup vs {label}", f"{result.speedup_over(label):.2f}x")
             for label in sorted(result.baselines) if result.speedup_over(label) is not None]
    if result.memory_bound:
        facts.append(("bandwidth", f"{result.gbps(best.median_ms):.1f} GB/s"))
    else:
        facts.append(("throughput", f"{result.tflops(best.median_ms):.1f} TFLOP/s"))
    facts.append(("arithmetic intensity",
                  f"{metrics.arithmetic_intensity(result.flops, result.bytes_moved):.1f} FLOP/byte"))
    w = 2 + max(len(k) for k, _ in facts)
    out.append("")
    out += [f"{(k + ':').ljust(w)}{v:>16}" for k, v in facts]
    if best.timing is not None and best.timing.at_timer_resolution:
        out.append("\nWarning: median latency is at event-timer resolution; "
                   "use a larger problem for a meaningful comparison.")
    return "\n".join(out)


@_command("tune", "search configurations for one problem",
          _compose(_operation_arguments(), lambda p: _timing_arguments(p), _storage_arguments,
                   _tune_arguments))
def _tune(session: _Session) -> int:
    from kernelforge.kernels import get_operator
    from kernelforge.tuning.search import search_space
    from kernelforge.tuning.tuner import Tuner

    args = session.args
    problem = build_problem(args.operation, args)
    if args.explain:
        from kernelforge.runtime.env import device_caps

        space = search_space(args.operation)
        if args.max_candidates is not None:
            space.max_candidates = args.max_candidates
        print(space.explain(problem, device_caps()))
        return 0
    operator = get_operator(args.operation)
    print(_problem_banner(problem) + "\n")
    tuner = Tuner(warmup=args.warmup, iterations=args.iterations, max_candidates=args.max_candidates,
                  measure_baselines=not args.no_baselines, flush_l2=not args.no_flush_l2,
                  db=session.db, cache=session.cache, log=print)
    result = tuner.tune(operator, problem, device=session.device)
    print(f"\nSearch space: {result.generated} grid points, {result.feasible} feasible, "
          f"{result.tested} measured in {result.elapsed_s:.1f}s")
    if args.show_all:
        print(_heading("All candidates"))
        for o in sorted(result.outcomes, key=lambda o: (not o.ok, o.timing.median_ms if o.timing else 0.0)):
            params = " ".join(f"{k}={v}" for k, v in o.config.items())
            if o.timing is None:
                print(f"  {o.status:>14}  {params}  {o.error[:120]}")
                continue
            text, _, _ = _rate(operator, problem, o.median_ms)
            print(f"  {o.timing.median_us:9.1f} us {text:>16}  {params}")
    print(_tuning_summary(result, operator))
    return 0 if result.best is not None else 1


# --- benchmark and compare ---------------------------------------------------------------
@dataclass
class _Evaluated:
    label: str
    status: str
    timing: object = None
    verification: object = None
    error: str = ""


def _evaluate(session: _Session, operator, problem: Problem, implementations: dict[str, Callable],
              reference, *, host_labels: frozenset = frozenset()) -> list[_Evaluated]:
    """Gate each implementation against ``reference``; time those that pass.

    Implementations in ``host_labels`` run on the CPU: they are timed with the
    host clock, unflushed, with at most 1 warmup call and 3 timed calls.
    """
    from kernelforge.benchmark.runner import benchmark
    from kernelforge.testing import verify

    args = session.args
    out = []
    for label, fn in implementations.items():
        try:
            check = verify(reference, fn().to(reference.device), dtype=problem.dtype)
        except Exception as exc:  # noqa: BLE001 -- reported per row, never fatal
            out.append(_Evaluated(label, "runtime_error", error=f"{type(exc).__name__}: {exc}"))
            continue
        if not check.passed:
            out.append(_Evaluated(label, "incorrect", verification=check, error=check.reason))
            continue
        on_host = label in host_labels
        timing = benchmark(fn, warmup=min(args.warmup, 1) if on_host else args.warmup,
                           iterations=min(args.iterations, 3) if on_host else args.iterations,
                           device="cpu" if on_host else session.device,
                           flush_l2=not (args.no_flush_l2 or on_host))
        out.append(_Evaluated(label, "ok", timing=timing, verification=check))
    return out


def _implementations(session: _Session, operator, problem: Problem, inputs, selection, *,
                     cpu: bool) -> dict[str, Callable]:
    impls = dict(operator.baselines(problem, inputs))
    impls[TUNED_LABEL] = lambda: operator.run(selection.config, *inputs)
    if cpu:
        host = tuple(t.detach().cpu() for t in inputs)
        impls["torch_cpu"] = lambda: operator.reference(*host)
    return impls


def _benchmark_arguments(p: argparse.ArgumentParser) -> None:
    p.add_argument("operation", choices=OPERATIONS)
    p.add_argument("--suite", default="sweep", choices=("smoke", "sweep", "transformer"))
    _timing_arguments(p, iterations=100)
    _storage_arguments(p)
    p.add_argument("--cpu-baseline", action="store_true",
                   help="also time torch eager on the host cores (label torch_cpu; 3 iterations)")


@_command("benchmark", "run a named workload suite", _benchmark_arguments)
def _benchmark(session: _Session) -> int:
    from kernelforge.benchmark import workloads
    from kernelforge.db import Measurement
    from kernelforge.kernels import get_operator
    from kernelforge.runtime.env import capture_environment
    from kernelforge.testing import exact_fp32_matmul

    args = session.args
    device = session.device
    operator = get_operator(args.operation)
    notes = f"benchmark:{args.suite}"
    print(capture_environment(device).render())
    print(_heading(f"{args.operation} / {args.suite} / {args.dtype}"))
    table = _Table([("shape", -24), ("impl", -14), ("config", -10), ("median ms", 11),
                    ("p99 ms", 10), ("metric", 16)])
    table.header()
    failures = 0
    for problem in workloads.problems(args.operation, args.suite, args.dtype):
        inputs = operator.make_inputs(problem, device)
        with exact_fp32_matmul():
            reference = operator.reference(*inputs)
            selection = session.select(operator, problem)
            impls = _implementations(session, operator, problem, inputs, selection,
                                     cpu=args.cpu_baseline)
            rows = _evaluate(session, operator, problem, impls, reference,
                             host_labels=frozenset({"torch_cpu"}))
        for row in rows:
            mine = row.label == TUNED_LABEL
            source = selection.source if mine else "-"
            config = selection.config if mine else None
            if row.status != "ok":
                failures += mine
                what = "INCORRECT" if row.status == "incorrect" else "failed"
                print(f"{problem.shape_key:<24}{row.label:<14}{source:<10}  {what}: {row.error[:100]}")
                session.record(notes, problem, Measurement(label=row.label, status=row.status,
                                                           config=config,
                                                           verification=row.verification,
                                                           error=row.error))
                continue
            text, tflops, gbps = _rate(operator, problem, row.timing.median_ms)
            table.row(problem.shape_key, row.label, source, f"{row.timing.median_ms:.4f}",
                      f"{row.timing.p99_ms:.4f}", text)
            session.record(notes, problem, Measurement(label=row.label, status="ok", config=config,
                                                       verification=row.verification,
                                                       timing=row.timing, tflops=tflops, gbps=gbps))
    return 1 if failures else 0


def _compare_arguments(p: argparse.ArgumentParser) -> None:
    _operation_arguments((*OPERATIONS, "transformer"))(p)
    _timing_arguments(p, iterations=100)
    _storage_arguments(p)
    p.add_argument("--batch", type=int, default=1, help="transformer: batch size")
    p.add_argument("--seq", type=int, default=2048, help="transformer: sequence length")
    p.add_argument("--hidden", type=int, default=4096, help="transformer: hidden size")
    p.add_argument("--heads", type=int, default=32, help="transformer: attention heads")
    p.add_argument("--intermediate", type=int, default=11008,
                   help="transformer: MLP intermediate size")


@_command("compare", "compare implementations at one shape, or a whole transformer block",
          _compare_arguments)
def _compare(session: _Session) -> int:
    args = session.args
    if args.operation == "transformer":
        return _compare_block(session)
    from kernelforge.kernels import get_operator
    from kernelforge.testing import exact_fp32_matmul

    operator = get_operator(args.operation)
    problem = build_problem(args.operation, args)
    device = session.device
    print(_problem_banner(problem))
    inputs = operator.make_inputs(problem, device)
    with exact_fp32_matmul():
        reference = operator.reference(*inputs)
        selection = session.select(operator, problem)
        print(f"config: {selection.describe()}")
        print(f"        {', '.join(f'{k}={v}' for k, v in selection.config.items())}")
        print(_heading("Comparison"))
        rows = _evaluate(session, operator, problem,
                         _implementations(session, operator, problem, inputs, selection, cpu=False),
                         reference)
    for row in rows:
        if row.status != "ok":
            print(f"{row.label}: {row.status.upper()} ({row.error[:120]})")
    timed = sorted((r for r in rows if r.status == "ok"), key=lambda r: r.timing.median_ms)
    eager = next((r.timing.median_ms for r in timed if r.label == "torch_eager"), None)
    table = _Table([("impl", -14), ("median ms", 11), ("p99 ms", 10), ("vs eager", 10),
                    ("metric", 16), ("max err", 11)])
    table.header()
    for r in timed:
        text, _, _ = _rate(operator, problem, r.timing.median_ms)
        ratio = f"{eager / r.timing.median_ms:.2f}x" if eager else "-"
        table.row(r.label, f"{r.timing.median_ms:.4f}", f"{r.timing.p99_ms:.4f}", ratio, text,
                  f"{r.verification.error:.2e}")
    return 0


def _compare_block(session: _Session) -> int:
    from kernelforge.integration import BlockConfig, benchmark_block

    args = session.args
    device = session.device
    block = BlockConfig(hidden=args.hidden, heads=args.heads, intermediate=args.intermediate)
    print(f"Transformer block: hidden={block.hidden} heads={block.heads} "
          f"intermediate={block.intermediate} batch={args.batch} seq={args.seq} dtype={args.dtype}")
    timings = benchmark_block(block, batch=args.batch, seq=args.seq, dtype=parse_dtype(args.dtype),
                              device=device, warmup=args.warmup, iterations=args.iterations,
                              cache=session.cache)
    print(_heading("Block latency"))
    base = timings["torch"].median_ms
    for backend, t in timings.items():
        ratio = "" if backend == "torch" else f"  ({base / t.median_ms:.3f}x)"
        print(f"{backend:<14}{t.median_ms:>10.3f} ms{ratio}")
    print("\nOnly the two RMSNorms and the MLP up-projection with its bias + GELU are swapped;\n"
          "attention and the other projections are PyTorch in both, so the block-level\n"
          "speedup is bounded by the share of block time those operators held.")
    return 0


# --- profile -----------------------------------------------------------------------------
def profile_child_argv(args: argparse.Namespace) -> list[str]:
    """Arguments of the one-launch child a counter profiler wraps.

    Rebuilt from the parsed arguments (not sliced from ``sys.argv``), so every
    shape flag reaches the child wherever it was written; the cache is passed
    through so the child picks the parent's configuration; nothing is recorded.
    """
    argv = ["profile", args.operation, "--dtype", args.dtype]
    for _, flag, _ in _SHAPES[args.operation]:
        value = getattr(args, flag, None)
        if value is not None:
            argv += [f"-{flag}" if len(flag) == 1 else f"--{flag}", str(value)]
    argv += ["--no-cache"] if args.no_cache else ["--cache", args.cache]
    return argv + ["--no-db", "--backend", "launch-once"]


#: The reference's name for the same function (its profiler was Nsight Compute).
nsight_child_argv = profile_child_argv


def _profile_arguments(p: argparse.ArgumentParser) -> None:
    from kernelforge.profiling.rocprof import DEFAULT_PASSES, PASSES

    _operation_arguments()(p)
    _timing_arguments(p, warmup=10, iterations=20)
    _storage_arguments(p)
    p.add_argument("--backend", default="torch", choices=("torch", "launch-once", "rocprof", "nsight"),
                   help="torch: kernel attribution via torch.profiler; rocprof: rocprofv3 counters "
                        "(MFMA utilisation, HBM traffic) of one launch; launch-once: the single "
                        "launch those counters wrap; nsight: NVIDIA only, reports unavailable")
    p.add_argument("--passes", nargs="+", default=list(DEFAULT_PASSES), choices=sorted(PASSES),
                   help="rocprof counter passes, one child run each")
    p.add_argument("--profile-dir", default=None,
                   help="rocprof output directory (default: a temporary directory)")


def _launch_once(session: _Session) -> int:
    """Warm the kernel up, flush the caches, then make the one launch that is measured."""
    import torch

    from kernelforge.benchmark.runner import flush_buffer
    from kernelforge.kernels import get_operator

    args = session.args
    device = session.device
    operator = get_operator(args.operation)
    problem = build_problem(args.operation, args)
    inputs = operator.make_inputs(problem, device)
    config = session.select(operator, problem).config
    operator.run(config, *inputs)
    flush_buffer(device).flush()
    operator.run(config, *inputs)
    torch.cuda.synchronize(device)
    from kernelforge.profiling.rocprof import CHILD_DONE

    print(CHILD_DONE, flush=True)  # the parent tells a finished child from one that died
    return 0


def _profile_rocprof(session: _Session) -> int:
    from kernelforge.kernels import get_operator
    from kernelforge.profiling import rocprof
    from kernelforge.runtime.env import MI355X_CAPS

    args = session.args
    if not rocprof.rocprof_available():
        print("rocprofv3 not found on PATH; it ships with ROCm in /opt/rocm/bin.", file=sys.stderr)
        return 2
    problem = build_problem(args.operation, args)
    operator = get_operator(args.operation)
    target = rocprof.self_command(profile_child_argv(args))
    with tempfile.TemporaryDirectory(prefix="kf_rocprof_") as scratch:
        out_dir = Path(args.profile_dir) if args.profile_dir else Path(scratch)
        result = rocprof.run(target, out_dir=out_dir, passes=tuple(args.passes))
    print(_problem_banner(problem))
    flops, moved = operator.flops(problem), operator.bytes_moved(problem)
    # fp32 products run on the fp32 MFMAs, a sixteenth of the 16-bit rate.
    peak = MI355X_CAPS.peak_fp32_tflops if problem.itemsize == 4 else MI355X_CAPS.peak_fp16_tflops
    # A product below the ridge point (peak FLOP/s over peak bytes/s, about
    # 315 FLOP/byte for 16-bit MFMA) is bandwidth-bound, e.g. a decode GEMV.
    ridge = peak * 1e3 / MI355X_CAPS.peak_hbm_gbps
    bound_by_hbm = operator.is_memory_bound() or flops < ridge * moved
    print(result.render(flops=flops, algorithmic_bytes=moved, peak_tflops=peak,
                        peak_gbps=MI355X_CAPS.peak_hbm_gbps, cu_count=MI355X_CAPS.cu_count,
                        memory_bound=bound_by_hbm))
    return 0 if result.ok else 1


@_command("profile", "attribute launches to kernels, or read hardware counters of one launch",
          _profile_arguments)
def _profile(session: _Session) -> int:
    args = session.args
    # Counter backends only assemble a command line here: the child does all
    # device work, so this process never opens the GPU.
    if args.backend == "nsight":
        print("ncu not found on PATH: Nsight Compute is NVIDIA's profiler; on MI355X use "
              "--backend rocprof.", file=sys.stderr)
        return 2
    if args.backend == "rocprof":
        return _profile_rocprof(session)
    if args.backend == "launch-once":
        return _launch_once(session)
    from kernelforge.kernels import get_operator
    from kernelforge.profiling import compare_launch_counts

    device = session.device
    operator = get_operator(args.operation)
    problem = build_problem(args.operation, args)
    inputs = operator.make_inputs(problem, device)
    selection = session.select(operator, problem)
    print(_problem_banner(problem))
    print(f"config: {selection.describe()}: {dict(selection.config)}")
    impls = dict(operator.baselines(problem, inputs))
    impls[TUNED_LABEL] = lambda: operator.run(selection.config, *inputs)
    print(_heading("Kernel attribution"))
    for profile in compare_launch_counts(impls, warmup=args.warmup, iterations=args.iterations):
        print(profile.render() + "\n")
    return 0


# --- report and cache --------------------------------------------------------------------
def _report_arguments(p: argparse.ArgumentParser) -> None:
    _storage_arguments(p)
    p.add_argument("--out", default="reports", help="output directory")


@_command("report", "render tables and figures from the database", _report_arguments)
def _report(session: _Session) -> int:
    from kernelforge.benchmark import report
    from kernelforge.db import ResultsDB

    path = Path(session.args.db)
    if not path.exists():
        print(f"no results database at {path}; run `kernelforge tune` first.", file=sys.stderr)
        return 2
    with ResultsDB(path) as db:
        n = db.counts()
        print(f"{n['results']} measurements across {n['problems']} problems and {n['runs']} runs")
        print(report.generate(db, session.args.out).render())
    return 0


def _cache_arguments(p: argparse.ArgumentParser) -> None:
    p.add_argument("cache_command", choices=("list", "clear"))
    _storage_arguments(p)


@_command("cache", "inspect or clear the tuned-config cache", _cache_arguments)
def _cache(session: _Session) -> int:
    from kernelforge.tuning.cache import ConfigCache

    cache = ConfigCache(session.args.cache)
    if session.args.cache_command == "clear":
        print(f"removed {cache.clear()} cached configuration(s) from {cache.path}")
        return 0
    entries = cache.entries()
    print(f"{cache.path}: {len(entries)} entry(ies)")
    for entry in entries:
        print(f"  {entry.describe()}")
    return 0


# --- entry point -------------------------------------------------------------------------
def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="kernelforge",
                                     description="Hardware-aware kernel autotuning on MI355X (gfx950).")
    parser.add_argument("--version", action="version", version=f"kernelforge {__version__}")
    sub = parser.add_subparsers(dest="command", required=True)
    for cmd in _REGISTRY.values():
        cmd.configure(sub.add_parser(cmd.name, help=cmd.help))
    return parser


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    try:
        with _Session(args) as session:
            return _REGISTRY[args.command].run(session)
    except KeyboardInterrupt:
        print("\ninterrupted", file=sys.stderr)
        return 130
    except (RuntimeError, ValueError) as exc:
        print(f"error: {exc}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    raise SystemExit(main())
