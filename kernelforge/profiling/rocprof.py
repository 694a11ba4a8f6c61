"""Hardware counters for one kernel launch, collected with ``rocprofv3``.

The event harness answers "how fast"; this answers "against what ceiling":
MFMA utilisation for the GEMMs and HBM bytes for the bandwidth-bound kernels,
each priced against the MI355X peak. It is this build's counterpart of the
reference's Nsight Compute wrapper (kernelforge/profiling/nsight.py:81-181):
the CLI re-runs itself as a child that makes exactly one measured launch
(``--backend launch-once``), under the profiler, and the parent parses what
the profiler wrote.

rocprofv3 does not split counters over replay passes: a pass may hold at
most 8 ``SQ_``, 4 ``TCC_`` (``FETCH_SIZE`` uses 3 of them and ``WRITE_SIZE``
2), 4 ``TCP_``, 2 ``TA_``, 2 ``TD_`` and 2 ``GRBM_`` counters, and a pass
that asks for more fails in ways that can stall. Every pass is checked
against those limits before anything runs (:func:`check_pass`), each pass is
its own child process, and each child runs under a time limit whose expiry
kills its whole process group. Durations come from a separate kernel-trace
pass, so counter collection never perturbs them.

Derived figures (:class:`LaunchCounters`):

* MFMA utilisation = ``SQ_VALU_MFMA_BUSY_CYCLES`` / (4 SIMDs x
  ``SQ_BUSY_CU_CYCLES``): the share of each SIMD's busy cycles its matrix
  core was busy; the shader clock = busy cycles per CU / kernel duration.
* HBM bytes = ``FETCH_SIZE`` x 2 + ``WRITE_SIZE`` x 1, in KiB. The factors
  are what the two counters read for a device copy of known size on MI355X
  (a 1 GiB copy reads 512 MiB of FETCH_SIZE and 1024 MiB of WRITE_SIZE).
  The counters see L2-to-fabric traffic, so Infinity Cache hits count as
  HBM bytes; gfx950 exposes no counter that separates the two.
"""

from __future__ import annotations

import csv
import os
import shutil
import signal
import subprocess
import sys
from collections import defaultdict
from dataclasses import dataclass, field
from pathlib import Path

#: Counter passes by name; each must fit one hardware pass (check_pass).
PASSES: dict[str, tuple[str, ...]] = {
    "trace": (),  # kernel trace only: durations, launch shape, registers
    "mfma": ("GRBM_GUI_ACTIVE", "SQ_BUSY_CU_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES",
             "SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
             "SQ_INSTS_VALU_MFMA_MOPS_F32"),
    "fetch": ("FETCH_SIZE",),
    "write": ("WRITE_SIZE",),
    "lds": ("SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_BUSY_CU_CYCLES"),
}
DEFAULT_PASSES = ("trace", "mfma", "fetch", "write")

#: Counters one pass may hold per hardware block, and the slots derived
#: counters occupy.
BLOCK_LIMITS = {"SQ": 8, "TCC": 4, "TCP": 4, "TA": 2, "TD": 2, "GRBM": 2}
_SLOTS = {"FETCH_SIZE": ("TCC", 3), "WRITE_SIZE": ("TCC", 2)}

#: Calibration of the traffic counters on MI355X (see module docstring).
FETCH_SCALE = 2.0
WRITE_SCALE = 1.0

SIMDS_PER_CU = 4
#: MFMA "MOPS" count 512 FLOPs each (one 16x16x32 16-bit MFMA is 16384 FLOPs, 32 MOPS).
FLOPS_PER_MOP = 512

#: The last line the launch-once child prints once its measured launch has
#: completed (cli/main.py); a pass whose log lacks it did not finish the program.
CHILD_DONE = "kernelforge launch-once: done"

#: Exit statuses of a process ended by SIGSEGV: as Popen reports it, and as a
#: shell would.
_SEGV = (-signal.SIGSEGV, 128 + signal.SIGSEGV)

#: Kernels of this library live in namespace ``kf``; the profiler reports
#: some names demangled (``void kf::...``) and others mangled (``_ZN2kf...``).
LIBRARY_KERNEL_MARKS = ("kf::", "_ZN2kf")


def is_library_kernel(name: str) -> bool:
    return any(mark in name for mark in LIBRARY_KERNEL_MARKS)


def rocprof_available() -> bool:
    return shutil.which("rocprofv3") is not None


def check_pass(counters: tuple[str, ...]) -> None:
    """Refuse a pass that exceeds one hardware pass on any block."""
    used: dict[str, int] = defaultdict(int)
    for name in counters:
        base = name.split("[")[0]
        for suffix in ("_sum", "_avr", "_min", "_max"):
            base = base.removesuffix(suffix)
        block, slots = _SLOTS.get(base, (base.split("_")[0], 1))
        used[block] += slots
    over = {b: n for b, n in used.items() if b in BLOCK_LIMITS and n > BLOCK_LIMITS[b]}
    if over:
        detail = ", ".join(f"{b} {n} > {BLOCK_LIMITS[b]}" for b, n in sorted(over.items()))
        raise ValueError(f"counter pass {list(counters)} exceeds one hardware pass: {detail}")


def build_command(target: list[str], *, counters: tuple[str, ...], out_dir: str | Path,
                  name: str) -> list[str]:
    """The rocprofv3 command line for one pass over ``target``.

    ``target`` must start with the program itself (``python ...``): the
    profiler's preloaded library initialises the GPU before the target runs,
    so a launcher in between (``env``, a shell) would re-exec a process that
    already holds the GPU.
    """
    check_pass(counters)
    mode = ["--pmc", *counters] if counters else ["--kernel-trace"]
    return ["rocprofv3", *mode, "--output-format", "csv", "-d", str(out_dir), "-o", name, "--",
            *target]


def self_command(argv: list[str]) -> list[str]:
    """This CLI, re-run with ``argv`` as a child process."""
    return [sys.executable, "-m", "kernelforge.cli.main", *argv]


@dataclass(frozen=True)
class Dispatch:
    """One kernel dispatch as the profiler saw it."""

    dispatch_id: int
    kernel: str
    grid: int
    workgroup: int
    lds_bytes: int
    vgprs: int
    agprs: int
    scratch_bytes: int
    start_ns: int
    end_ns: int
    counters: dict[str, float] = field(default_factory=dict)

    @property
    def duration_us(self) -> float:
        return (self.end_ns - self.start_ns) / 1e3


def _int(row: dict[str, str], *keys: str) -> int:
    for key in keys:
        if row.get(key) not in (None, ""):
            return int(float(row[key]))
    return 0


def parse_counter_csv(path: str | Path) -> list[Dispatch]:
    """``*_counter_collection.csv``: one row per (dispatch, counter)."""
    rows: dict[int, dict] = {}
    values: dict[int, dict[str, float]] = defaultdict(dict)
    with open(path, newline="") as handle:
        for row in csv.DictReader(handle):
            did = _int(row, "Dispatch_Id")
            rows.setdefault(did, row)
            values[did][row["Counter_Name"]] = float(row["Counter_Value"])
    return [Dispatch(did, r["Kernel_Name"], _int(r, "Grid_Size"), _int(r, "Workgroup_Size"),
                     _int(r, "LDS_Block_Size"), _int(r, "VGPR_Count"), _int(r, "Accum_VGPR_Count"),
                     _int(r, "Scratch_Size"), _int(r, "Start_Timestamp"), _int(r, "End_Timestamp"),
                     values[did])
            for did, r in sorted(rows.items())]


def parse_trace_csv(path: str | Path) -> list[Dispatch]:
    """``*_kernel_trace.csv``: one row per dispatch."""
    out = []
    with open(path, newline="") as handle:
        for r in csv.DictReader(handle):
            grid = _int(r, "Grid_Size_X") * max(1, _int(r, "Grid_Size_Y")) * max(1, _int(r, "Grid_Size_Z"))
            wg = _int(r, "Workgroup_Size_X") * max(1, _int(r, "Workgroup_Size_Y")) * max(1, _int(r, "Workgroup_Size_Z"))
            out.append(Dispatch(_int(r, "Dispatch_Id"), r["Kernel_Name"], grid, wg,
                                _int(r, "LDS_Block_Size"), _int(r, "VGPR_Count"),
                                _int(r, "Accum_VGPR_Count"), _int(r, "Scratch_Size"),
                                _int(r, "Start_Timestamp"), _int(r, "End_Timestamp")))
    return sorted(out, key=lambda d: d.dispatch_id)


def measured_dispatch(dispatches: list[Dispatch]) -> Dispatch | None:
    """The launch-once child's measured launch: its last dispatch of a library kernel
    (the child warms the kernel up once before flushing the caches and measuring)."""
    ours = [d for d in dispatches if is_library_kernel(d.kernel)]
    return ours[-1] if ours else None


def allocated_vgprs(vgpr_count: int) -> int:
    """Vector registers a gfx950 wave is given, from rocprofv3's ``VGPR_Count``.

    The kernel descriptor holds the allocation as a count of 8-register
    granules; rocprofv3 multiplies that count by 4, so on gfx950 its field
    reads half the allocation. Checked against the ``.vgpr_count`` of this
    library's own code objects: 223 and 256 registers (the 128x256 and
    256x256 GEMM tiles) read 112 and 128, 56 and 79 (softmax and RMSNorm
    rows) read 28 and 40.
    """
    return 2 * vgpr_count


@dataclass
class LaunchCounters:
    """Counters and derived figures of one launch, merged over the passes."""

    kernel: str = ""
    grid: int = 0
    workgroup: int = 0
    lds_bytes: int = 0
    vgprs: int = 0
    agprs: int = 0
    scratch_bytes: int = 0
    duration_us: float | None = None
    counters: dict[str, float] = field(default_factory=dict)

    def absorb(self, d: Dispatch, *, timed: bool) -> None:
        self.kernel, self.grid, self.workgroup = d.kernel, d.grid, d.workgroup
        self.lds_bytes, self.vgprs, self.agprs, self.scratch_bytes = (
            d.lds_bytes, d.vgprs, d.agprs, d.scratch_bytes)
        if timed:
            self.duration_us = d.duration_us
        self.counters.update(d.counters)

    @property
    def mfma_utilisation(self) -> float | None:
        busy, mfma = self.counters.get("SQ_BUSY_CU_CYCLES"), self.counters.get("SQ_VALU_MFMA_BUSY_CYCLES")
        if not busy or mfma is None:
            return None
        return mfma / (SIMDS_PER_CU * busy)

    def shader_clock_ghz(self, cu_count: int) -> float | None:
        busy = self.counters.get("SQ_BUSY_CU_CYCLES")
        if not busy or not self.duration_us:
            return None
        return busy / cu_count / (self.duration_us * 1e3)

    @property
    def mfma_flops(self) -> float | None:
        mops = [v for k, v in self.counters.items() if k.startswith("SQ_INSTS_VALU_MFMA_MOPS_")]
        return sum(mops) * FLOPS_PER_MOP if mops else None

    @property
    def hbm_bytes(self) -> float | None:
        fetch, write = self.counters.get("FETCH_SIZE"), self.counters.get("WRITE_SIZE")
        if fetch is None or write is None:
            return None
        return (FETCH_SCALE * fetch + WRITE_SCALE * write) * 1024.0


@dataclass
class RocprofRun:
    """The passes of one profile: their commands, status codes and the merged launch.

    ``returncodes`` are the passes' verdicts; ``raw_returncodes`` what each
    rocprofv3 process actually returned. The two differ only where rocprofv3
    itself ended on SIGSEGV after the profiled program had printed its
    completion line and the pass's output held the measured launch: that pass
    is usable, and ``notes`` says what happened so that ``render`` prints it.
    """

    commands: list[list[str]]
    returncodes: list[int]
    launch: LaunchCounters | None
    log: str = ""
    raw_returncodes: list[int] = field(default_factory=list)
    notes: list[str] = field(default_factory=list)

    @property
    def ok(self) -> bool:
        return self.launch is not None and all(rc == 0 for rc in self.returncodes)

    def render(self, *, flops: int, algorithmic_bytes: int, peak_tflops: float,
               peak_gbps: float, cu_count: int, memory_bound: bool) -> str:
        lines = [f"$ {' '.join(c)}" for c in self.commands]
        lines += [f"note: {n}" for n in self.notes]
        if self.launch is None:
            lines.append("no dispatch of a library kernel was recorded")
            if self.log.strip():
                lines.append(self.log.strip()[-2000:])
            return "\n".join(lines)
        c = self.launch
        rows = [("kernel", c.kernel[:100]), ("grid / workgroup", f"{c.grid} / {c.workgroup} lanes"),
                ("VGPR / AGPR / scratch",
                 f"{allocated_vgprs(c.vgprs)} / {c.agprs} / {c.scratch_bytes} B "
                 f"(VGPR_Count {c.vgprs} x 2)"),
                ("LDS", f"{c.lds_bytes} B")]
        if c.duration_us:
            rows.append(("duration", f"{c.duration_us:.1f} us"))
            tflops = flops / (c.duration_us * 1e-6) / 1e12
            gbps = algorithmic_bytes / (c.duration_us * 1e-6) / 1e9
            rows.append(("achieved (algorithmic)",
                         f"{tflops:.1f} TFLOP/s = {100 * tflops / peak_tflops:.1f}% of peak; "
                         f"{gbps:.0f} GB/s = {100 * gbps / peak_gbps:.1f}% of HBM"))
        if c.mfma_utilisation is not None:
            clock = c.shader_clock_ghz(cu_count)
            rows.append(("MFMA busy", f"{100 * c.mfma_utilisation:.1f}% of SIMD busy cycles"
                         + (f" at {clock:.2f} GHz" if clock else "")))
        if c.mfma_flops:
            rows.append(("MFMA FLOPs", f"{c.mfma_flops:.4g} (model: {flops:.4g})"))
        if c.hbm_bytes is not None:
            text = f"{c.hbm_bytes / 2**20:.1f} MiB = {c.hbm_bytes / max(algorithmic_bytes, 1):.2f}x algorithmic"
            if c.duration_us:
                gbps = c.hbm_bytes / (c.duration_us * 1e-6) / 1e9
                text += f"; {gbps:.0f} GB/s = {100 * gbps / peak_gbps:.1f}% of HBM"
            rows.append(("HBM traffic", text))
        for name in sorted(c.counters):
            rows.append((name, f"{c.counters[name]:,.0f}"))
        width = max(len(k) for k, _ in rows)
        lines.append("")
        lines += [f"{k.ljust(width)}  {v}" for k, v in rows]
        lines.append("bound: " + ("HBM" if memory_bound else "MFMA"))
        return "\n".join(lines)


def _run_pass(command: list[str], timeout: float) -> tuple[int, str]:
    proc = subprocess.Popen(command, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                            start_new_session=True)
    try:
        out, _ = proc.communicate(timeout=timeout)
        return proc.returncode, out
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        out, _ = proc.communicate()
        return -signal.SIGKILL, out + f"\n[killed after {timeout:.0f} s]"


def run(target: list[str], *, out_dir: str | Path, passes: tuple[str, ...] = DEFAULT_PASSES,
        timeout: float = 120.0) -> RocprofRun:
    """Profile ``target`` once per pass and merge the measured launch's figures."""
    if not rocprof_available():
        raise RuntimeError("rocprofv3 was not found on PATH; it ships with ROCm (/opt/rocm/bin)")
    unknown = sorted(set(passes) - set(PASSES))
    if unknown:
        raise ValueError(f"unknown counter passes {unknown}; available: {sorted(PASSES)}")
    root = Path(out_dir)
    commands, codes, raw, logs, notes = [], [], [], [], []
    launch = LaunchCounters()
    found = False
    for name in passes:
        pass_dir = root / name
        command = build_command(target, counters=PASSES[name], out_dir=pass_dir, name=name)
        commands.append(command)
        rc, log = _run_pass(command, timeout)
        logs.append(log)
        pattern = "*_counter_collection.csv" if PASSES[name] else "*_kernel_trace.csv"
        files = sorted(pass_dir.rglob(pattern))
        parse = parse_counter_csv if PASSES[name] else parse_trace_csv
        measured = measured_dispatch(parse(files[-1])) if files else None
        raw.append(rc)
        # rocprofv3 can end on SIGSEGV in its own teardown, after the program it
        # ran has exited and its output files are written. Such a pass is used,
        # and reported, only if the program got to its last line and the
        # measured launch is in the output; any other signal or exit status
        # fails the profile.
        finished = CHILD_DONE in log
        if rc in _SEGV and measured is not None and finished:
            codes.append(0)
            notes.append(f"pass '{name}': rocprofv3 exited on SIGSEGV (status {rc}) after the "
                         "profiled program printed its completion line; the pass's output holds "
                         "the measured launch and is used")
        else:
            codes.append(rc)
            if rc in _SEGV:
                notes.append(f"pass '{name}': rocprofv3 exited on SIGSEGV (status {rc}) "
                             + ("before the profiled program finished" if not finished
                                else "with no measured launch in its output"))
        if measured is None and rc == 0:
            codes[-1] = 1  # ran, but recorded no launch of this library
        if codes[-1] != 0:
            break  # a failed pass ends the profile: nothing further runs on the GPU
        launch.absorb(measured, timed=not PASSES[name])
        found = True
    return RocprofRun(commands, codes, launch if found else None, "\n".join(logs), raw, notes)
