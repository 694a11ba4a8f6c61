"""Benchmark the hot path on one MI355X and print ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one launch of a kernel over one batch of synthetic input that is
already resident in HBM. Every BASELINE configuration is measured; the
headline ``value`` is configuration 3, the fp16 GEMM 2048x4096x4096 in
TFLOP/s (BASELINE.json ``metric``). Two further lines cover the kernels
added beyond the BASELINE set: vector_add over 2^26 fp32 elements (the HBM
probe) and the two-pass RMSNorm on fp16 rows of 32768.

Timing, as the reference measures (kernelforge/benchmark/runner.py:169-183):
for each of the K steps, flush L2 + Infinity Cache, record a start event,
launch, record an end event, all on the stream the kernel runs on; K steps
are bracketed by synchronisation. Throughput is the algorithmic work (FLOP or
minimum bytes) divided by the mean event-timed step, priced against the
MI355X peak. The per-launch events add a few microseconds of dispatch gap to
every step, so short kernels read slower than their rocprofv3 durations.

Beside it, ``sustained_*`` reports back-to-back throughput: the inputs are
held in R copies whose combined size is at least twice L2 + Infinity Cache,
and the K steps (step i uses copy i mod R and keeps its own output) are
captured into one HIP graph whose replay is event-timed. That removes host
launch cost but keeps the dependency drain between consecutive kernels and
the clock the GPU holds under sustained load. Each replay's outputs are
checked bitwise against the eager outputs. After every configuration, a soak
replays the headline GEMM's graph back to back for ``--soak-seconds`` (8 by
default) and reports its per-launch time as ``soak`` on that configuration:
the GPU busy without a gap for seconds, at its sustained clock. The amdgpu
driver's own busy percentage (sysfs ``gpu_busy_percent``) is sampled every
0.1 s meanwhile and reported beside it.

The torch comparators (hipBLASLt, the unfused matmul + bias + GELU, torch's
GEMV, ``a + b``, eager RMSNorm) are timed the same way but alternating step by
step with the kernel they are compared to (``interleaved_us`` is that
kernel's mean in the same run), so a ratio of the two is not skewed by the
clock rising or falling between two runs. Per configuration the order is:
correctness gate, interleaved comparison, then the configuration's own W
warm-up and K timed steps (the comparison's launches precede them).

Each configuration's output is checked against torch on the same device with
the reference's gate before it is timed. The CPU baseline is the oracle
(oracle/ops.py, torch eager in fp32) timed on the host cores over each full
workload, with the reference's CPU warm-up and iteration counts.

``roofline.kernel_us`` / ``kernel_frac`` and ``roofline.traffic`` come from the
committed rocprofv3 summaries in profiles/ (kernelforge.profiling.bench_profiles
over a ``--marks`` run of this script); each is null, with the reason, when the
summary was made from another library build (source digest) or another
configuration than the one dispatch picks in this run.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "fp16 GEMM TFLOP/s @2048x4096x4096; RMSNorm/softmax/GEMV HBM GB/s"


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


#: Rotation span of the input copies: twice L2 (32 MiB) + Infinity Cache (256 MiB).
ROTATION_BYTES = 2 * (32 + 256) * 2**20


def _copies(step_bytes: int) -> int:
    """Input copies whose combined size covers the rotation span (at least 2)."""
    return max(2, -(-ROTATION_BYTES // step_bytes))


def _time_flushed(fn, steps: int, warmup: int, flush) -> list[float]:
    """The reference's method: flush, event, launch, event -- per step (ms)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        flush.flush()
        start[i].record()
        fn()
        end[i].record()
    torch.cuda.synchronize()
    return [start[i].elapsed_time(end[i]) for i in range(steps)]


def _time_interleaved(ours, theirs, steps: int, warmup: int, flush) -> tuple[list[float], list[float]]:
    """The reference's per-step method for a kernel and its torch comparator, the
    two alternating step by step (ms per step of each).

    Timed one after the other, the second would run further into the clock ramp
    that sustained MFMA load causes on this board (a fused-linear launch takes
    400+ us early in a process and 340 us once the clock settles), which biases
    a ratio of the two; alternating gives both the same clock.
    """
    import torch

    for _ in range(warmup):
        ours()
        theirs()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for i in range(steps):
        flush.flush()
        ev[i][0].record()
        ours()
        ev[i][1].record()
        flush.flush()
        ev[i][2].record()
        theirs()
        ev[i][3].record()
    torch.cuda.synchronize()
    return ([ev[i][0].elapsed_time(ev[i][1]) for i in range(steps)],
            [ev[i][2].elapsed_time(ev[i][3]) for i in range(steps)])


def _time_graph(fns, steps: int, warmup: int, flush):
    """Mean ms per step of `steps` launches captured into one HIP graph.

    ``fns[i]`` runs the step on input copy i and returns its output; step j
    uses copy j mod len(fns). Returns (ms_per_step, max relative deviation of
    the replay's outputs from eager outputs of the same copies).
    """
    import torch

    n = len(fns)
    eager = [fns[i]() for i in range(n)]  # also warms every code path before capture
    for i in range(warmup):
        fns[i % n]()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [fns[j % n]() for j in range(steps)]  # every output stays live
    torch.cuda.synchronize()
    # The untimed replay, the flush and the timed replay are queued back to back:
    # a host wait between them would leave the GPU idle, and MFMA-heavy launches
    # after an idle period run at a lower clock for their first milliseconds.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    graph.replay()  # untimed replay
    flush.flush()
    start.record()
    graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    dev = 0.0
    for j in range(min(steps, n)):
        ref = eager[j].float()
        scale = float(ref.abs().max()) or 1.0
        dev = max(dev, float((outs[j].float() - ref).abs().max()) / scale)
    del graph, outs, eager
    return ms, dev


def _soak(fns, seconds: float, steps: int) -> dict:
    """Back-to-back replays of one graph of ``steps`` launches for about ``seconds``.

    ``fns[i]`` runs the step on input copy i and returns its output, as in
    ``_time_graph``. The GPU runs this one kernel without a gap for the whole
    window, long enough for a utilisation sampler outside the process to see it
    and for the board to reach its sustained power and clock. The host waits
    for every batch of replays, so the queue stays short. After the window the
    last replay's outputs are checked bitwise against eager runs of the same
    copies.
    """
    import torch

    n = len(fns)
    eager = [fns[i]() for i in range(n)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [fns[j % n]() for j in range(steps)]
    graph.replay()
    torch.cuda.synchronize()
    batch = max(1, 2000 // steps)  # about 2000 launches per host wait
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    replays = 0
    t0 = time.perf_counter()
    start.record()
    while time.perf_counter() - t0 < seconds:
        for _ in range(batch):
            graph.replay()
        replays += batch
        torch.cuda.synchronize()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    for j in range(min(steps, n)):
        if not torch.equal(outs[j], eager[j]):
            raise RuntimeError(f"soak: replay output {j} differs from the eager result")
    launches = replays * steps
    ms = start.elapsed_time(end)
    del graph, outs, eager
    return {"launches": launches, "gpu_seconds": ms / 1e3, "wall_seconds": wall,
            "us_per_launch": ms * 1e3 / launches}


def _busy_path(dev) -> Path | None:
    """The amdgpu driver's busy-percentage file of ``dev`` in sysfs, if readable."""
    import torch

    p = torch.cuda.get_device_properties(dev)
    path = Path(f"/sys/bus/pci/devices/{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:"
                f"{p.pci_device_id:02x}.0/gpu_busy_percent")
    try:
        int(path.read_text().strip())
    except (OSError, ValueError):
        return None
    return path


class _BusySampler:
    """Reads the GPU's busy percentage every ``period`` seconds on a thread."""

    def __init__(self, path: Path, period: float = 0.1):
        import threading

        self.path, self.period = path, period
        self.samples: list[int] = []
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)

    def _run(self) -> None:
        while not self._stop.wait(self.period):
            try:
                self.samples.append(int(self.path.read_text().strip()))
            except (OSError, ValueError):
                pass

    def __enter__(self):
        self._thread.start()
        return self

    def __exit__(self, *exc) -> None:
        self._stop.set()
        self._thread.join()

    def summary(self) -> dict:
        n = len(self.samples)
        return {"source": str(self.path), "period_s": self.period, "samples": n,
                "mean_pct": sum(self.samples) / n if n else None,
                "min_pct": min(self.samples) if n else None}


def profile_entry(path: Path, name: str, config: dict | None, digest: str) -> tuple[dict | None, str | None]:
    """The committed rocprofv3 summary of workload ``name`` (``profiles/kernel_trace.json``
    or ``profiles/hbm_traffic.json``, written by kernelforge.profiling.bench_profiles), or
    None and the reason it does not describe this run: no entry, another library build
    (source digest), or a configuration dispatch no longer picks."""
    if not path.exists():
        return None, f"{path.name} is missing"
    doc = json.loads(path.read_text())
    entry = doc.get("kernels", {}).get(name)
    if entry is None:
        return None, f"{path.name} has no entry for {name}"
    if doc.get("library_digest") != digest:
        return None, (f"{path.name} profiled library sources {doc.get('library_digest')}, "
                      f"this run loaded {digest}")
    if entry.get("config") != config:
        return None, (f"{path.name} profiled configuration {entry.get('config')}, "
                      f"dispatch picked {config} in this run")
    return entry, None


def _kernel_time(name: str, work: float, scale: float, peak: float, config: dict | None,
                 digest: str) -> dict:
    """Median kernel duration of ``name``'s kernel from the committed rocprofv3 trace and
    the roofline fraction it gives; null, with the reason, when that trace does not
    describe the kernel this run launched."""
    entry, why = profile_entry(REPO / "profiles" / "kernel_trace.json", name, config, digest)
    if entry is None:
        return {"kernel_us": None, "kernel_frac": None, "kernel_method": None, "kernel_null_reason": why}
    us = float(entry["median_us"])
    return {"kernel_us": us, "kernel_frac": (work / (us * 1e-6)) / scale / peak,
            "kernel_name": entry["kernel"], "kernel_grid": entry["grid"],
            "kernel_method": "median dispatch duration in profiles/kernel_trace.json (rocprofv3 "
                             "kernel trace of this library build and configuration)"}


def _traffic(name: str, config: dict | None, digest: str) -> tuple[float | None, str | None]:
    """HBM bytes per launch of ``name``'s kernel from the committed FETCH_SIZE/WRITE_SIZE
    summary (copy-calibrated), or None and the reason."""
    entry, why = profile_entry(REPO / "profiles" / "hbm_traffic.json", name, config, digest)
    return (None, why) if entry is None else (float(entry["traffic_bytes"]), None)


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-sustained", action="store_true",
                        help="skip the graph-captured sustained runs and the soak (profiling the "
                             "headline method)")
    parser.add_argument("--marks", default=None,
                        help="launch a marker kernel before each workload and write the workload "
                             "list, configurations and library digest to this file, for "
                             "kernelforge.profiling.bench_profiles to cut a rocprofv3 run into "
                             "workloads")
    parser.add_argument("--soak-seconds", type=float, default=8.0,
                        help="seconds of back-to-back headline GEMM launches after the configs "
                             "(0 skips)")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build has no multi-GPU path (every GPU box here has "
            "one GPU). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import numpy as np
    import torch

    from kernelforge.benchmark import metrics
    from kernelforge.benchmark.runner import flush_buffer
    from kernelforge.kernels.fused_linear import fused_linear_gelu, linear_gelu_reference
    from kernelforge.kernels.matmul import matmul
    from kernelforge.kernels.rmsnorm import rmsnorm, rmsnorm_reference
    from kernelforge.kernels.softmax import softmax
    from kernelforge.runtime.env import device_caps, host_cores
    from kernelforge.testing import assert_verified, exact_fp32_matmul

    from kernelforge.kernels import get_operator
    from kernelforge.profiling.bench_profiles import MARKER_STRIDE
    from kernelforge.runtime import hip
    from kernelforge.runtime.dispatch import select_config
    from kernelforge.tuning.config import Problem

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    caps = device_caps(dev)
    flush = flush_buffer(dev)
    steps, warmup = args.steps, args.warmup
    g = torch.Generator().manual_seed(0)
    results: dict[str, dict] = {}
    digest = hip.source_digest()
    marks: list[dict] = []

    def mark(name, config, **extra):
        """With --marks: an int8 fill of a size of its own ahead of the workload's
        launches (the marker bench_profiles cuts a profile at), and its entry."""
        if args.marks is None:
            return
        torch.full((MARKER_STRIDE * (len(marks) + 1),), 77, dtype=torch.int8, device=dev)
        marks.append({"name": name, "config": config, **extra})

    def pick(operation, dtype, **dims):
        """The config dispatch would run: user cache, packaged winners, default."""
        sel = select_config(get_operator(operation), Problem.create(operation, dtype, **dims),
                            device=dev)
        return sel.config, {"config_source": sel.source, "kernel_config": dict(sel.config)}

    def record(name, fns, work, unit, peak, extra=None):
        scale = 1e12 if unit == "TFLOP/s" else 1e9
        config = (extra or {}).get("kernel_config")
        traffic, traffic_why = _traffic(name, config, digest)
        flushed = _time_flushed(fns[0], steps, warmup, flush)
        mean_ms = float(np.mean(flushed))
        rate = (work / (mean_ms * 1e-3)) / scale
        if args.no_sustained:
            sustained_ms, replay_diff = float("nan"), 0.0
        else:
            sustained_ms, replay_diff = _time_graph(fns, steps, warmup, flush)
        if replay_diff != 0.0:
            raise RuntimeError(f"{name}: graph replay differs from the eager result by {replay_diff:.3g}")
        entry = {
            "value": rate,
            "unit": unit,
            "mean_us": mean_ms * 1e3,
            "median_us": float(np.median(flushed)) * 1e3,
            "min_us": float(np.min(flushed)) * 1e3,
            "sustained_us": sustained_ms * 1e3,
            "sustained_value": (work / (sustained_ms * 1e-3)) / scale,
            "sustained_copies": len(fns),
            "work": work,
            "roofline": {
                "bound": "mfma" if unit == "TFLOP/s" else "hbm",
                "achieved": rate,
                "peak": peak,
                "unit": "TFLOP/s" if unit == "TFLOP/s" else "GB/s",
                "frac": rate / peak,
                "traffic": traffic,
                # Kernel time without the per-launch dispatch gap: the median
                # kernel duration of the same workload in the committed rocprofv3
                # kernel trace (profiles/kernel_trace.json), if it profiled this
                # library build and this configuration.
                **_kernel_time(name, work, scale, peak, config, digest),
            },
        }
        if traffic is None:
            entry["roofline"]["traffic_null_reason"] = traffic_why
        if extra:
            entry.update(extra)
        results[name] = entry
        _log(f"{name}: {rate:.1f} {unit} ({entry['roofline']['frac'] * 100:.1f}% of peak), "
             f"mean {mean_ms * 1e3:.1f} us; sustained {sustained_ms * 1e3:.1f} us/step over "
             f"{len(fns)} copies")
        return entry

    def copies_of(step_bytes, *tensors):
        """R device copies of each tensor (R from the rotation span)."""
        r = _copies(step_bytes)
        return r, [[t.clone() for t in tensors] for _ in range(r)]

    hbm = caps.peak_hbm_gbps
    f16_peak = caps.peak_fp16_tflops

    # --- inputs: every configuration's seeded data, in HBM before anything is timed --
    # Generating a configuration's inputs on the host right before timing it would
    # leave the GPU idle for hundreds of milliseconds, and the first launches after
    # an idle period run at a lower clock while it ramps back up (measured on the
    # fused linear: 400-450 us for the first 10-20 launches, 340 us after).
    x = torch.randn(4096, 4096, generator=g)
    gamma = 1.0 + 0.1 * torch.randn(4096, generator=g)
    dx, dgamma = x.to(dev), gamma.to(dev)
    soft = {}
    soft_host = {}  # the CPU baseline runs on the same inputs
    for cols in (4096, 11008):
        s = 3.0 * torch.randn(8192, cols, generator=g)
        s[torch.randperm(8192, generator=g)[:82]] += 60.0
        soft_host[cols] = s.to(torch.float16)
        soft[cols] = soft_host[cols].to(dev)
        del s
    M, N, K = 2048, 4096, 4096
    a = (torch.randn(M, K, generator=g) / K**0.5).to(torch.float16).to(dev)
    b = (torch.randn(K, N, generator=g) / K**0.5).to(torch.float16).to(dev)
    FM, FN, FK = 4096, 11008, 4096
    fx_host = (torch.randn(FM, FK, generator=g) / FK**0.5).to(torch.float16)
    fw_host = (torch.randn(FK, FN, generator=g) / FK**0.5).to(torch.float16)
    fb_host = (0.02 * torch.randn(FN, generator=g)).to(torch.float16)
    fx, fw, fb = fx_host.to(dev), fw_host.to(dev), fb_host.to(dev)
    vx = (torch.rand(1, 4096, generator=g) * 2 - 1).to(torch.bfloat16).to(dev)
    vw = (torch.rand(4096, 11008, generator=g) * 2 - 1).to(torch.bfloat16).to(dev)
    VN = 1 << 26
    va_host = torch.randn(VN, generator=g)
    vb_host = torch.randn(VN, generator=g)
    va, vb = va_host.to(dev), vb_host.to(dev)
    WR, WC = 4096, 32768
    wx = torch.randn(WR, WC, generator=g).to(torch.float16).to(dev)
    wg = (1.0 + 0.1 * torch.randn(WC, generator=g)).to(torch.float16).to(dev)
    torch.cuda.synchronize()

    # --- calibration: a plain device-to-device copy of 1 GiB (read + write) -----
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = [torch.empty_like(src) for _ in range(2)]
    mark("hbm_copy_1GiB", None, kernel_hint="copy", copy_bytes=src.numel() * 4,
         algorithmic_bytes=2 * src.numel() * 4)
    record("hbm_copy_1GiB", [lambda i=i: dst[i].copy_(src) for i in range(2)],
           2 * src.numel() * 4, "GB/s", hbm)
    del src, dst

    # --- config 1: RMSNorm fp32 [4096,4096], eps=1e-6 ----------------------------
    cfg, src = pick("rmsnorm", "fp32", rows=4096, cols=4096)
    mark("rmsnorm_fp32_4096x4096", src["kernel_config"],
         algorithmic_bytes=metrics.rmsnorm_bytes(4096, 4096, 4))
    assert_verified(rmsnorm_reference(dx, dgamma, eps=1e-6),
                    rmsnorm(dx, dgamma, eps=1e-6, config=cfg), context="rmsnorm config 1")
    work = metrics.rmsnorm_bytes(4096, 4096, 4)
    r, cp = copies_of(work, dx, dgamma)
    record("rmsnorm_fp32_4096x4096",
           [lambda c=c: rmsnorm(c[0], c[1], eps=1e-6, config=cfg) for c in cp],
           work, "GB/s", hbm, src)
    del cp

    # --- config 2: softmax fp16 [8192,4096] and [8192,11008], 1% rows +60 ---------
    for cols in (4096, 11008):
        ds = soft.pop(cols)
        cfg, src = pick("softmax", "fp16", rows=8192, cols=cols)
        mark(f"softmax_fp16_8192x{cols}", src["kernel_config"],
             algorithmic_bytes=metrics.softmax_bytes(8192, cols, 2))
        out = softmax(ds, config=cfg)
        assert torch.isfinite(out).all()
        assert_verified(torch.softmax(ds.float(), -1), out, dtype=torch.float16,
                        context=f"softmax config 2 ({cols})")
        work = metrics.softmax_bytes(8192, cols, 2)
        r, cp = copies_of(work, ds)
        record(f"softmax_fp16_8192x{cols}",
               [lambda c=c, cfg=cfg: softmax(c[0], config=cfg) for c in cp],
               work, "GB/s", hbm, src)
        del ds, cp, out

    # --- config 3: GEMM fp16 2048x4096x4096 (headline) -----------------------------
    gcfg, src = pick("matmul", "fp16", M=M, N=N, K=K)
    mark("gemm_fp16_2048x4096x4096", src["kernel_config"],
         algorithmic_bytes=metrics.matmul_bytes(M, N, K, 2))
    with exact_fp32_matmul():
        assert_verified(torch.matmul(a.float(), b.float()), matmul(a, b, config=gcfg),
                        dtype=torch.float16, context="gemm config 3")
    mine, tg = _time_interleaved(lambda: matmul(a, b, config=gcfg), lambda: torch.matmul(a, b),
                                 steps, warmup, flush)
    r, cp = copies_of((M * K + K * N + M * N) * 2, a, b)
    gemm = record("gemm_fp16_2048x4096x4096",
                  [lambda c=c: matmul(c[0], c[1], config=gcfg) for c in cp],
                  metrics.matmul_flops(M, N, K), "TFLOP/s", f16_peak, src)
    gemm["torch_hipblaslt_tflops"] = metrics.matmul_flops(M, N, K) / (np.mean(tg) * 1e-3) / 1e12
    gemm["interleaved_us"] = float(np.mean(mine)) * 1e3
    gemm["speedup_vs_hipblaslt"] = float(np.mean(tg)) / float(np.mean(mine))
    ms, _ = (float("nan"), 0.0) if args.no_sustained else _time_graph([lambda c=c: torch.matmul(c[0], c[1]) for c in cp], steps, warmup, flush)
    gemm["torch_hipblaslt_sustained_tflops"] = metrics.matmul_flops(M, N, K) / (ms * 1e-3) / 1e12
    del cp

    # --- config 4: fused linear fp16 4096x11008x4096 + bias + GELU(tanh) -----------
    fcfg, src = pick("fused_linear", "fp16", M=FM, N=FN, K=FK)
    mark("fused_linear_fp16_4096x11008x4096", src["kernel_config"],
         algorithmic_bytes=metrics.fused_linear_bytes(FM, FN, FK, 2, fused=True))
    assert_verified(linear_gelu_reference(fx, fw, fb), fused_linear_gelu(fx, fw, fb, config=fcfg),
                    context="fused linear config 4")
    mine, tu = _time_interleaved(lambda: fused_linear_gelu(fx, fw, fb, config=fcfg),
                                 lambda: linear_gelu_reference(fx, fw, fb), steps, warmup, flush)
    r, cp = copies_of(metrics.fused_linear_bytes(FM, FN, FK, 2, fused=True), fx, fw, fb)
    fused = record("fused_linear_fp16_4096x11008x4096",
                   [lambda c=c: fused_linear_gelu(c[0], c[1], c[2], config=fcfg) for c in cp],
                   metrics.matmul_flops(FM, FN, FK), "TFLOP/s", f16_peak, src)
    fused["unfused_torch_3op_us"] = float(np.mean(tu)) * 1e3
    fused["interleaved_us"] = float(np.mean(mine)) * 1e3
    fused["speedup_vs_unfused"] = float(np.mean(tu)) / float(np.mean(mine))
    ms, _ = (float("nan"), 0.0) if args.no_sustained else _time_graph([lambda c=c: linear_gelu_reference(c[0], c[1], c[2]) for c in cp],
                        steps, warmup, flush)
    fused["unfused_torch_3op_sustained_us"] = ms * 1e3
    del fx, fw, cp

    # --- config 5a: decode GEMV bf16 1x11008x4096 ----------------------------------
    vcfg, src = pick("matmul", "bf16", M=1, N=11008, K=4096)
    mark("gemv_bf16_1x11008x4096", src["kernel_config"],
         algorithmic_bytes=metrics.matmul_bytes(1, 11008, 4096, 2))
    assert_verified(torch.matmul(vx.float(), vw.float()), matmul(vx, vw, config=vcfg),
                    dtype=torch.bfloat16, context="gemv config 5a")
    work = metrics.matmul_bytes(1, 11008, 4096, 2)
    mine, tv = _time_interleaved(lambda: matmul(vx, vw, config=vcfg), lambda: torch.matmul(vx, vw),
                                 steps, warmup, flush)
    r, cp = copies_of(work, vx, vw)
    gemv = record("gemv_bf16_1x11008x4096",
                  [lambda c=c: matmul(c[0], c[1], config=vcfg) for c in cp],
                  work, "GB/s", hbm, src)
    gemv["torch_gbps"] = work / (np.mean(tv) * 1e-3) / 1e9
    gemv["interleaved_us"] = float(np.mean(mine)) * 1e3
    ms, _ = (float("nan"), 0.0) if args.no_sustained else _time_graph([lambda c=c: torch.matmul(c[0], c[1]) for c in cp], steps, warmup, flush)
    gemv["torch_sustained_gbps"] = work / (ms * 1e-3) / 1e9
    del cp

    # --- widened rows: vector_add (the HBM probe) and the two-pass RMSNorm --------
    from kernelforge.kernels.vector_add import vector_add

    acfg, src = pick("vector_add", "fp32", n=VN)
    mark("vector_add_fp32_67108864", src["kernel_config"],
         algorithmic_bytes=metrics.vector_add_bytes(VN, 4))
    assert torch.equal(vector_add(va, vb, config=acfg), va + vb), "vector_add must be bit-exact"
    work = metrics.vector_add_bytes(VN, 4)
    mine, ta = _time_interleaved(lambda: vector_add(va, vb, config=acfg), lambda: va + vb, steps,
                                 warmup, flush)
    r, cp = copies_of(work, va, vb)
    vadd = record("vector_add_fp32_67108864",
                  [lambda c=c: vector_add(c[0], c[1], config=acfg) for c in cp],
                  work, "GB/s", hbm, src)
    vadd["torch_gbps"] = work / (np.mean(ta) * 1e-3) / 1e9
    vadd["interleaved_us"] = float(np.mean(mine)) * 1e3
    del cp, va, vb

    wcfg, src = pick("rmsnorm", "fp16", rows=WR, cols=WC)
    mark(f"rmsnorm_two_pass_fp16_{WR}x{WC}", src["kernel_config"],
         algorithmic_bytes=metrics.rmsnorm_bytes(WR, WC, 2))
    assert_verified(rmsnorm_reference(wx, wg, eps=1e-6), rmsnorm(wx, wg, eps=1e-6, config=wcfg),
                    context="two-pass rmsnorm")
    work = metrics.rmsnorm_bytes(WR, WC, 2)
    mine, tw = _time_interleaved(lambda: rmsnorm(wx, wg, eps=1e-6, config=wcfg),
                                 lambda: rmsnorm_reference(wx, wg, eps=1e-6), steps, warmup, flush)
    r, cp = copies_of(work, wx, wg)
    wide = record(f"rmsnorm_two_pass_fp16_{WR}x{WC}",
                  [lambda c=c: rmsnorm(c[0], c[1], eps=1e-6, config=wcfg) for c in cp],
                  work, "GB/s", hbm, src)
    wide["torch_eager_gbps"] = work / (np.mean(tw) * 1e-3) / 1e9
    wide["interleaved_us"] = float(np.mean(mine)) * 1e3
    del cp

    # --- soak: the headline GEMM back to back for a few seconds --------------------
    if not args.no_sustained and args.soak_seconds > 0:
        _log(f"soak: gemm_fp16_2048x4096x4096 back to back for {args.soak_seconds:.0f} s")
        r, cp = copies_of((M * K + K * N + M * N) * 2, a, b)
        fns = [lambda c=c: matmul(c[0], c[1], config=gcfg) for c in cp]
        path = _busy_path(dev)
        if path is None:
            soak = _soak(fns, args.soak_seconds, steps)
            soak["gpu_busy"] = None
        else:
            with _BusySampler(path) as sampler:
                soak = _soak(fns, args.soak_seconds, steps)
            soak["gpu_busy"] = sampler.summary()
        soak["value"] = metrics.matmul_flops(M, N, K) / (soak["us_per_launch"] * 1e-6) / 1e12
        soak["unit"] = "TFLOP/s"
        gemm["soak"] = soak
        _log(f"soak: {soak['launches']} launches, {soak['us_per_launch']:.1f} us each = "
             f"{soak['value']:.1f} TFLOP/s")
        del cp

    # --- CPU baseline: the oracle on the host cores, full workloads ----------------
    # The reference's CPU timing (kernelforge/benchmark/runner.py:153-166): perf_counter
    # around each call after the warm-up, median of the calls; 1 warm-up and 3 calls
    # for the GEMM and the fused linear, 3 and 20 for the row kernels, the GEMV and
    # vector_add. Same seeded inputs as the GPU run, every workload at full size.
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import ops

        cores = host_cores()
        torch.set_num_threads(cores)

        def cpu_entry(fn, work, unit, sample, warmup, iterations):
            for _ in range(warmup):
                fn()
            secs = []
            for _ in range(iterations):
                t0 = time.perf_counter()
                fn()
                secs.append(time.perf_counter() - t0)
            med = float(np.median(secs))
            scale = 1e12 if unit == "TFLOP/s" else 1e9
            _log(f"cpu baseline: {sample}: {med * 1e3:.1f} ms per call on {cores} threads")
            return {"value": work / med / scale, "unit": unit, "cores": cores, "kind": "port",
                    "timer": "perf_counter", "median_ms": med * 1e3,
                    "sample": f"{sample}, full workload; median of {iterations} calls after "
                              f"{warmup} warm-up"}

        ca, cb = a.cpu(), b.cpu()
        cpu = cpu_entry(lambda: ops.matmul_ref(ca, cb), metrics.matmul_flops(M, N, K), "TFLOP/s",
                        f"oracle matmul_ref (torch fp32 on CPU), {M}x{N}x{K} fp16 inputs", 1, 3)
        results["gemm_fp16_2048x4096x4096"]["cpu_baseline"] = cpu
        del ca, cb
        results["fused_linear_fp16_4096x11008x4096"]["cpu_baseline"] = cpu_entry(
            lambda: ops.linear_gelu_ref(fx_host, fw_host, fb_host), metrics.matmul_flops(FM, FN, FK),
            "TFLOP/s", f"oracle linear_gelu_ref, {FM}x{FN}x{FK} fp16 inputs", 1, 3)
        results["rmsnorm_fp32_4096x4096"]["cpu_baseline"] = cpu_entry(
            lambda: ops.rmsnorm_ref(x, gamma, 1e-6), metrics.rmsnorm_bytes(4096, 4096, 4), "GB/s",
            "oracle rmsnorm_ref, [4096,4096] fp32", 3, 20)
        for cols in (4096, 11008):
            cs = soft_host[cols]
            results[f"softmax_fp16_8192x{cols}"]["cpu_baseline"] = cpu_entry(
                lambda cs=cs: ops.softmax_ref(cs), metrics.softmax_bytes(8192, cols, 2), "GB/s",
                f"oracle softmax_ref, [8192,{cols}] fp16 with the +60 rows", 3, 20)
        cvx, cvw = vx.cpu(), vw.cpu()
        results["gemv_bf16_1x11008x4096"]["cpu_baseline"] = cpu_entry(
            lambda: ops.matmul_ref(cvx, cvw), metrics.matmul_bytes(1, 11008, 4096, 2), "GB/s",
            "oracle matmul_ref, 1x11008x4096 bf16", 3, 20)
        results["vector_add_fp32_67108864"]["cpu_baseline"] = cpu_entry(
            lambda: ops.vector_add_ref(va_host, vb_host), metrics.vector_add_bytes(VN, 4), "GB/s",
            f"oracle vector_add_ref, {VN} fp32 elements", 3, 20)
        cwx, cwg = wx.cpu(), wg.cpu()
        results[f"rmsnorm_two_pass_fp16_{WR}x{WC}"]["cpu_baseline"] = cpu_entry(
            lambda: ops.rmsnorm_ref(cwx, cwg, 1e-6), metrics.rmsnorm_bytes(WR, WC, 2), "GB/s",
            f"oracle rmsnorm_ref, [{WR},{WC}] fp16", 3, 20)

    if args.marks is not None:
        Path(args.marks).parent.mkdir(parents=True, exist_ok=True)
        Path(args.marks).write_text(json.dumps({"library_digest": digest, "argv": sys.argv,
                                                "workloads": marks}, indent=1) + "\n")
        _log(f"marks: {len(marks)} workloads -> {args.marks}")

    line = {
        "metric": METRIC,
        "value": gemm["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": gemm["mean_us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "gemm_fp16_2048x4096x4096",
            "M": M,
            "N": N,
            "K": K,
            "device": caps.name,
            "arch": caps.gcn_arch,
            "flush_bytes": caps.flush_bytes,
        },
        "roofline": gemm["roofline"],
        "cpu_baseline": cpu,
        "configs": results,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
