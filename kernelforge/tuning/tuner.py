"""Tune one problem: candidates -> availability -> gate -> time -> rank -> persist.

The guarantees are the reference's (kernelforge/tuning/tuner.py:1-370):

* **Nothing incorrect is ranked.** Every candidate passes the correctness gate
  (:mod:`kernelforge.testing`) before it may be timed; a wrong answer is
  recorded with its error and never timed.
* **Gating and timing are separate passes.** All candidates are gated first,
  then the survivors are timed back to back under identical settings, so no
  candidate's timing shares the GPU with another candidate's setup.
* **Ranking is on the median**, and failures are classified, recorded and
  kept out of the ranking.

How this build differs from a JIT tuner. Every configuration here is an
ahead-of-time instantiation in ``libkernelforge_hip.so``. An operator can
therefore say *before launching* whether a candidate exists
(:meth:`Operator.availability`, backed by the library's variant table); a
missing one is recorded as ``compile_error`` without touching the GPU. A
launch that fails returns a ``KF_ERR_*`` status that the binding raises as a
typed exception carrying the code, and the code decides the outcome:

=========================================  ================
``KF_ERR_NOT_BUILT``, ``KF_ERR_OUT_OF_RESOURCES``  ``compile_error``
``KF_ERR_OUT_OF_MEMORY``                     ``out_of_memory``
any other code                               ``runtime_error``
=========================================  ================

Exceptions from elsewhere (torch, a Python operator) have no code and fall
back to the reference's rule on the class name: ``...OutOfMemory...`` is an
OOM, ``...OutOfResources...``/``...Compil...``/``...Resource...`` a compile
error, anything else a runtime error.

Each candidate moves through the pipeline as a mutable :class:`_Trial`; the
result exposes frozen :class:`CandidateOutcome` records.
"""

from __future__ import annotations

import time
from collections import Counter
from collections.abc import Callable
from dataclasses import dataclass, field

import torch

from kernelforge.benchmark import metrics
from kernelforge.benchmark.runner import DEFAULT_ITERATIONS, DEFAULT_WARMUP, TimingResult, benchmark
from kernelforge.db import Measurement, ResultsDB
from kernelforge.kernels.base import Operator
from kernelforge.runtime import hip
from kernelforge.runtime.env import Environment, capture_environment, device_caps, require_gpu
from kernelforge.testing import VerificationResult, exact_fp32_matmul, verify
from kernelforge.tuning.cache import ConfigCache
from kernelforge.tuning.config import KernelConfig, Problem

#: Candidate outcomes; only ``ok`` is ranked.
STATUS_OK = "ok"
STATUS_COMPILE_ERROR = "compile_error"
STATUS_RUNTIME_ERROR = "runtime_error"
STATUS_INCORRECT = "incorrect"
STATUS_OOM = "out_of_memory"

#: The label tuned candidates carry in the results database.
TUNED_LABEL = "kernelforge"

_ERROR_CHARS = 400

_BY_CODE = {
    hip.KF_ERR_NOT_BUILT: STATUS_COMPILE_ERROR,
    hip.KF_ERR_OUT_OF_RESOURCES: STATUS_COMPILE_ERROR,
    hip.KF_ERR_OUT_OF_MEMORY: STATUS_OOM,
}


def _status_by_name(name: str) -> str:
    if "OutOfMemory" in name:
        return STATUS_OOM
    if any(tag in name for tag in ("OutOfResources", "Compil", "Resource")):
        return STATUS_COMPILE_ERROR
    return STATUS_RUNTIME_ERROR


def _classify(exc: BaseException) -> tuple[str, str]:
    """(status, one-line message) for an exception a candidate raised."""
    name = type(exc).__name__
    text = " ".join(str(exc).split())[:_ERROR_CHARS]
    if isinstance(exc, hip.KernelError) and exc.code:
        status = _BY_CODE.get(exc.code, STATUS_RUNTIME_ERROR)
    else:
        status = _status_by_name(name)
    return status, (text if status == STATUS_OOM else f"{name}: {text}")


@dataclass(frozen=True)
class CandidateOutcome:
    config: KernelConfig
    status: str
    verification: VerificationResult | None = None
    timing: TimingResult | None = None
    error: str = ""

    @property
    def ok(self) -> bool:
        return self.status == STATUS_OK

    @property
    def median_ms(self) -> float:
        if self.timing is None:
            raise ValueError(f"candidate {self.config!r} has no timing ({self.status})")
        return self.timing.median_ms


@dataclass
class _Trial:
    """One candidate on its way through the pipeline."""

    config: KernelConfig
    status: str = STATUS_OK
    verification: VerificationResult | None = None
    timing: TimingResult | None = None
    error: str = ""

    def fail(self, status: str, error: str) -> None:
        self.status, self.error, self.timing = status, error, None

    def freeze(self) -> CandidateOutcome:
        return CandidateOutcome(self.config, self.status, self.verification, self.timing,
                                self.error)


@dataclass
class TuningResult:
    problem: Problem
    environment: Environment
    generated: int
    feasible: int
    outcomes: tuple[CandidateOutcome, ...]
    baselines: dict[str, TimingResult]
    flops: int
    bytes_moved: int
    elapsed_s: float
    memory_bound: bool = False
    rejections: tuple[tuple[KernelConfig, str], ...] = field(default=(), repr=False)

    @property
    def tested(self) -> int:
        """Candidates that reached the gate (available ones plus AOT misses)."""
        return len(self.outcomes)

    @property
    def correct(self) -> int:
        return sum(o.ok for o in self.outcomes)

    def ranked(self) -> list[CandidateOutcome]:
        """Correct candidates by median latency, fastest first (never by the minimum,
        which rewards the luckiest sample)."""
        return sorted(filter(lambda o: o.ok, self.outcomes), key=lambda o: o.median_ms)

    @property
    def best(self) -> CandidateOutcome | None:
        return next(iter(self.ranked()), None)

    @property
    def best_config(self) -> KernelConfig | None:
        return None if self.best is None else self.best.config

    def tflops(self, ms: float) -> float:
        return metrics.tflops(self.flops, ms)

    def gbps(self, ms: float) -> float:
        return metrics.gbps(self.bytes_moved, ms)

    def speedup_over(self, label: str) -> float | None:
        base, best = self.baselines.get(label), self.best
        if base is None or best is None:
            return None
        return metrics.speedup(base.median_ms, best.median_ms)

    def status_counts(self) -> dict[str, int]:
        return dict(Counter(o.status for o in self.outcomes))


class Tuner:
    """Runs the pipeline for any :class:`~kernelforge.kernels.base.Operator`."""

    def __init__(
        self,
        *,
        warmup: int = DEFAULT_WARMUP,
        iterations: int = DEFAULT_ITERATIONS,
        flush_l2: bool = True,
        max_candidates: int | None = None,
        measure_baselines: bool = True,
        seed: int = 0,
        db: ResultsDB | None = None,
        cache: ConfigCache | None = None,
        log: Callable[[str], None] | None = None,
    ) -> None:
        self.warmup = warmup
        self.iterations = iterations
        self.flush_l2 = flush_l2
        self.max_candidates = max_candidates
        self.measure_baselines = measure_baselines
        self.seed = seed
        self.db = db
        self.cache = cache
        self._sink = log

    def log(self, message: str) -> None:
        if self._sink is not None:
            self._sink(message)

    def _time(self, fn: Callable[[], object], device: torch.device) -> TimingResult:
        return benchmark(fn, warmup=self.warmup, iterations=self.iterations, device=device,
                         flush_l2=self.flush_l2)

    # --- the pipeline -----------------------------------------------------------------
    def tune(self, operator: Operator, problem: Problem, *,
             device: torch.device | str | None = None) -> TuningResult:
        began = time.perf_counter()
        dev = torch.device(device) if device is not None else require_gpu()
        env = capture_environment(dev)
        plan = operator.search_space().generate(problem, device_caps(dev),
                                                max_candidates=self.max_candidates)
        trials = [_Trial(config) for config in plan]
        inputs = operator.make_inputs(problem, dev, seed=self.seed)
        # One numerical policy for candidates and baselines alike: fp32
        # references and torch baselines at full fp32 precision.
        with exact_fp32_matmul():
            reference = operator.reference(*inputs)
            self.log(f"Verifying candidates... ({len(trials)} to check)")
            for trial in trials:
                self._gate(operator, problem, trial, inputs, reference)
            self.log(f"{sum(t.status == STATUS_OK for t in trials)} / {len(trials)} "
                     "configurations passed correctness")
            self.log("Benchmarking...")
            for trial in trials:
                if trial.status == STATUS_OK:
                    self._measure(operator, trial, inputs, dev)
            baselines = (self._baselines(operator, problem, inputs, reference, dev)
                         if self.measure_baselines else {})
        result = TuningResult(
            problem=problem,
            environment=env,
            generated=plan.generated,
            feasible=plan.feasible,
            outcomes=tuple(t.freeze() for t in trials),
            baselines=baselines,
            flops=operator.flops(problem),
            bytes_moved=operator.bytes_moved(problem),
            elapsed_s=time.perf_counter() - began,
            memory_bound=operator.is_memory_bound(),
            rejections=plan.rejected,
        )
        self._store_winner(result)
        self._record(result)
        return result

    def _gate(self, operator: Operator, problem: Problem, trial: _Trial,
              inputs: tuple[torch.Tensor, ...], reference: torch.Tensor) -> None:
        missing = operator.availability(trial.config, problem)
        if missing:
            trial.fail(STATUS_COMPILE_ERROR, missing)
            return
        try:
            output = operator.run(trial.config, *inputs)
        except Exception as exc:  # one bad candidate must not end the sweep
            trial.fail(*_classify(exc))
            return
        trial.verification = verify(reference, output, dtype=problem.dtype)
        if not trial.verification.passed:
            trial.fail(STATUS_INCORRECT, trial.verification.reason)

    def _measure(self, operator: Operator, trial: _Trial, inputs: tuple[torch.Tensor, ...],
                 device: torch.device) -> None:
        try:
            trial.timing = self._time(lambda: operator.run(trial.config, *inputs), device)
        except Exception as exc:
            trial.fail(*_classify(exc))

    def _baselines(self, operator: Operator, problem: Problem, inputs: tuple[torch.Tensor, ...],
                   reference: torch.Tensor, device: torch.device) -> dict[str, TimingResult]:
        """Each comparison implementation, gated like a candidate, then timed
        with the candidates' warmup, iterations and flush."""
        timed: dict[str, TimingResult] = {}
        for label, fn in operator.baselines(problem, inputs).items():
            try:
                check = verify(reference, fn(), dtype=problem.dtype)
                if check.passed:
                    timed[label] = self._time(fn, device)
                else:
                    self.log(f"  baseline {label} disagrees with the reference: {check.reason}")
            except Exception as exc:
                self.log(f"  baseline {label} unavailable: {_classify(exc)[1]}")
        return timed

    # --- persistence ------------------------------------------------------------------
    def _store_winner(self, result: TuningResult) -> None:
        best = result.best
        if self.cache is None or best is None:
            return
        self.cache.put(result.problem, result.environment.device_key, best.config,
                       median_us=best.timing.median_us if best.timing else None,
                       timestamp=result.environment.timestamp,
                       candidates_tested=result.tested)

    def _record(self, result: TuningResult) -> None:
        if self.db is None:
            return
        from kernelforge import __version__

        def rates(timing: TimingResult | None) -> dict[str, float | None]:
            if timing is None:
                return {"tflops": None, "gbps": None}
            return {"tflops": result.tflops(timing.median_ms), "gbps": result.gbps(timing.median_ms)}

        rows = [Measurement(label=TUNED_LABEL, status=o.status, config=o.config,
                            verification=o.verification, timing=o.timing, error=o.error,
                            **rates(o.timing))
                for o in result.outcomes]
        rows += [Measurement(label=label, status=STATUS_OK, timing=t, **rates(t))
                 for label, t in result.baselines.items()]
        run_id = self.db.start_run(result.environment, notes="tune", version=__version__)
        self.db.record_many(run_id, result.problem, rows)
