"""Reports from the results database: ``summary.md``, one CSV per operation, figures.

Every number a reader sees is read back from a database row and carries the
provenance of the run that measured it (kernelforge/benchmark/report.py:
263-364 defines the same artefacts), so regenerating after a new benchmark
never leaves a stale figure. Only timed rows whose verification did not fail
are used: a fast but wrong measurement never reaches a table or a chart.

Built here as plain Python over the database's own queries, with matplotlib
for the figures and nothing else:

* the fastest usable row per (operation, dtype, shape, label) is picked in
  one pass over the rows; problems are ordered by their element count, so
  ``512x512x512`` comes before ``2048x4096x4096``;
* each table row carries the MI355X roofline fraction of the tuned
  (``kernelforge``) measurement -- GB/s over 8 TB/s for the memory-bound
  operators, TFLOP/s over the dense MFMA peak of the dtype otherwise -- and
  its speedup over ``torch_eager``;
* the labels are this build's: ``torch_cpu`` (torch eager on the host cores),
  ``torch_eager`` (hipBLASLt / ATen-HIP), ``hip_default`` (the fixed default
  configuration) and ``kernelforge`` (the tuned one);
* a database that mixes flushed with unflushed rows, or GPU event timings
  with host-clock ones, gets a warning instead of a silent ranking.
"""

from __future__ import annotations

import csv
import json
from collections import defaultdict
from dataclasses import dataclass, field
from math import prod
from pathlib import Path
from typing import Any

from kernelforge.db import ResultsDB
from kernelforge.runtime.env import MI355X_CAPS

#: Order of implementations in tables and legends; unknown labels follow, sorted.
LABEL_ORDER = ("torch_cpu", "torch_eager", "hip_default", "kernelforge")

LABEL_TITLES = {
    "torch_cpu": "PyTorch CPU",
    "torch_eager": "PyTorch eager (ROCm)",
    "hip_default": "HIP default config",
    "kernelforge": "kernelforge (tuned)",
}

#: The label whose throughput and roofline fraction the tables report.
TUNED_LABEL = "kernelforge"

MEMORY_BOUND_OPERATIONS = frozenset({"rmsnorm", "softmax", "vector_add"})

#: The GPU timer; rows with another timer are host-clock measurements.
GPU_TIMER = "hip_event"

_CSV_FIELDS = ("operation", "dtype", "shape_key", "label", "median_us", "mean_us", "p99_us",
               "tflops", "gbps", "size", "timer", "flushed_l2", "params_json", "run_id")


@dataclass
class ReportArtifacts:
    directory: Path
    summary: Path
    figures: list[Path] = field(default_factory=list)
    tables: list[Path] = field(default_factory=list)
    notes: list[str] = field(default_factory=list)

    def render(self) -> str:
        lines = [f"Report written to {self.directory}", f"  {self.summary.name}"]
        lines += [f"  {p.name}" for p in (*self.tables, *self.figures)]
        lines += [f"  note: {note}" for note in self.notes]
        return "\n".join(lines)


def _pyplot() -> Any:
    try:
        import matplotlib
    except ImportError as exc:  # pragma: no cover - depends on the install
        raise RuntimeError("report figures need matplotlib") from exc
    matplotlib.use("Agg")
    import matplotlib.pyplot as plt

    return plt


def _usable(db: ResultsDB) -> list[dict]:
    """Timed rows whose verification did not fail, with their element count."""
    out = []
    for row in db.rows():
        if row["median_us"] is None or row["correct"] == 0:
            continue
        row["size"] = prod(json.loads(row["dims_json"]).values())
        row["params"] = json.loads(row["params_json"]) if row["params_json"] else {}
        out.append(row)
    return out


def _fastest(rows: list[dict]) -> dict[tuple[str, str, str, str], dict]:
    """The fastest row per (operation, dtype, shape, label); ties keep the earlier."""
    best: dict[tuple[str, str, str, str], dict] = {}
    for row in rows:
        key = (row["operation"], row["dtype"], row["shape_key"], row["label"])
        if key not in best or row["median_us"] < best[key]["median_us"]:
            best[key] = row
    return best


def _ordered_labels(labels) -> list[str]:
    present = set(labels)
    return [x for x in LABEL_ORDER if x in present] + sorted(present - set(LABEL_ORDER))


def _problems(fastest: dict, operation: str) -> list[tuple[str, str, int]]:
    """(shape, dtype, size) of an operation's problems, smallest first."""
    seen = {(k[2], k[1], r["size"]) for k, r in fastest.items() if k[0] == operation}
    return sorted(seen, key=lambda p: (p[2], p[1], p[0]))


def _peak(operation: str, dtype: str) -> tuple[str, float]:
    if operation in MEMORY_BOUND_OPERATIONS:
        return "gbps", MI355X_CAPS.peak_hbm_gbps
    if dtype == "fp32":
        return "tflops", MI355X_CAPS.peak_fp32_tflops
    return "tflops", MI355X_CAPS.peak_fp16_tflops


def _cell(row: dict | None) -> str:
    return "-" if row is None else f"{row['median_us']:.1f}"


def _table(fastest: dict, operation: str) -> list[str]:
    problems = _problems(fastest, operation)
    labels = _ordered_labels(k[3] for k in fastest if k[0] == operation)
    unit = "GB/s" if operation in MEMORY_BOUND_OPERATIONS else "TFLOP/s"
    header = (["shape", "dtype"] + [f"{LABEL_TITLES.get(x, x)} (us)" for x in labels]
              + [f"{LABEL_TITLES[TUNED_LABEL]} {unit}", "of MI355X peak", "speedup vs eager"])
    lines = ["| " + " | ".join(header) + " |", "|" + " --- |" * len(header)]
    for shape, dtype, _ in problems:
        row_of = {x: fastest.get((operation, dtype, shape, x)) for x in labels}
        cells = [shape, dtype] + [_cell(row_of[x]) for x in labels]
        mine, eager = row_of.get(TUNED_LABEL), row_of.get("torch_eager")
        column, peak = _peak(operation, dtype)
        rate = None if mine is None else mine.get(column)
        cells += [f"{rate:.1f}", f"{100.0 * rate / peak:.1f}%"] if rate is not None else ["-", "-"]
        cells.append(f"{eager['median_us'] / mine['median_us']:.2f}x" if mine and eager else "-")
        lines.append("| " + " | ".join(cells) + " |")
    return lines


def _environment(db: ResultsDB) -> list[str]:
    runs = db.runs()
    if not runs:
        return ["No runs recorded."]
    latest = runs[-1]
    fields = (("GPU", "gpu_name"), ("Architecture", "gpu_arch"), ("Compute units", "cu_count"),
              ("HIP", "hip_version"), ("Driver", "driver_version"), ("PyTorch", "torch_version"),
              ("kernelforge", "kernelforge_version"), ("Recorded", "timestamp"))
    return ["| Field | Value |", "| --- | --- |"] + [
        f"| {title} | {latest.get(key) or '-'} |" for title, key in fields]


def _warnings(rows: list[dict]) -> list[str]:
    notes = []
    flushed = sum(1 for r in rows if r["flushed_l2"] == 1)
    if 0 < flushed < len(rows):
        notes.append(
            f"this database mixes {flushed} cache-flushed measurement(s) with "
            f"{len(rows) - flushed} unflushed; the unflushed rows report a bandwidth the kernel "
            "would not see on cold inputs, so the two are not comparable")
    timers = sorted({r["timer"] for r in rows})
    if len(timers) > 1:
        notes.append(f"this database mixes timers ({', '.join(timers)}); only {GPU_TIMER} rows "
                     "are GPU measurements")
    return notes


def _write_csv(path: Path, fastest: dict, operation: str) -> Path:
    order = {(s, d): i for i, (s, d, _) in enumerate(_problems(fastest, operation))}
    rows = sorted((r for k, r in fastest.items() if k[0] == operation),
                  key=lambda r: (order[(r["shape_key"], r["dtype"])], r["label"]))
    with open(path, "w", newline="") as handle:
        writer = csv.DictWriter(handle, fieldnames=_CSV_FIELDS, extrasaction="ignore")
        writer.writeheader()
        writer.writerows(rows)
    return path


def _bars(plt, fastest: dict, operation: str, *, value: str, ylabel: str, title: str,
          path: Path) -> Path:
    problems = _problems(fastest, operation)
    two_dtypes = len({d for _, d, _ in problems}) > 1
    ticks = [f"{s} {d}" if two_dtypes else s for s, d, _ in problems]
    labels = _ordered_labels(k[3] for k in fastest if k[0] == operation)
    width = 0.8 / max(1, len(labels))
    fig, ax = plt.subplots(figsize=(max(7.0, 1.1 * len(problems) + 2.5), 4.2))
    for i, label in enumerate(labels):
        heights = []
        for shape, dtype, _ in problems:
            row = fastest.get((operation, dtype, shape, label))
            heights.append(float("nan") if row is None or row.get(value) is None else row[value])
        ax.bar([j + i * width for j in range(len(problems))], heights, width=width,
               label=LABEL_TITLES.get(label, label))
    ax.set_xticks([j + 0.4 - width / 2 for j in range(len(problems))])
    ax.set_xticklabels(ticks, rotation=45, ha="right", fontsize=8)
    ax.set_ylabel(ylabel)
    ax.set_title(title)
    ax.legend(fontsize=8)
    ax.grid(axis="y", alpha=0.3)
    fig.tight_layout()
    fig.savefig(path, dpi=140)
    plt.close(fig)
    return path


def _heatmap(plt, rows: list[dict], path: Path) -> Path | None:
    """Best tuned latency over the BLOCK_M x BLOCK_N plane, for the GEMM problem
    (shape and dtype) with the most tuned candidates: what each tile can do at
    best over the other parameters, never an average across dtypes."""
    tuned = [r for r in rows if r["operation"] == "matmul" and r["label"] == TUNED_LABEL
             and "BLOCK_M" in r["params"] and "BLOCK_N" in r["params"]]
    if not tuned:
        return None
    per_problem: dict[tuple[str, str], list[dict]] = defaultdict(list)
    for r in tuned:
        per_problem[(r["shape_key"], r["dtype"])].append(r)
    (shape, dtype), chosen = max(per_problem.items(), key=lambda kv: (len(kv[1]), kv[0]))
    best: dict[tuple[int, int], float] = {}
    for r in chosen:
        tile = (r["params"]["BLOCK_M"], r["params"]["BLOCK_N"])
        best[tile] = min(best.get(tile, float("inf")), r["median_us"])
    ms = sorted({t[0] for t in best})
    ns = sorted({t[1] for t in best})
    grid = [[best.get((m, n), float("nan")) for n in ns] for m in ms]
    fig, ax = plt.subplots(figsize=(5.6, 4.4))
    image = ax.imshow(grid, cmap="viridis_r", aspect="auto")
    ax.set_xticks(range(len(ns)), [str(n) for n in ns])
    ax.set_yticks(range(len(ms)), [str(m) for m in ms])
    ax.set_xlabel("BLOCK_N")
    ax.set_ylabel("BLOCK_M")
    ax.set_title(f"Best median latency by tile ({shape} {dtype})")
    for i, line in enumerate(grid):
        for j, v in enumerate(line):
            if v == v:
                ax.text(j, i, f"{v:.0f}", ha="center", va="center", color="white", fontsize=7)
    fig.colorbar(image, ax=ax, label="median latency (us)")
    fig.tight_layout()
    fig.savefig(path, dpi=140)
    plt.close(fig)
    return path


def generate(db: ResultsDB, directory: str | Path = "reports", *,
             operations: list[str] | None = None) -> ReportArtifacts:
    """Write ``summary.md``, ``<operation>.csv`` and the figures into ``directory``."""
    out = Path(directory)
    out.mkdir(parents=True, exist_ok=True)
    art = ReportArtifacts(directory=out, summary=out / "summary.md")
    rows = _usable(db)
    if not rows:
        art.summary.write_text(
            "# kernelforge results\n\nNo correct, timed measurements in the database yet. "
            "Run `python -m kernelforge tune` or `python -m kernelforge benchmark` first.\n")
        art.notes.append("database contained no usable measurements")
        return art
    plt = _pyplot()
    fastest = _fastest(rows)
    lines = [
        "# kernelforge results", "",
        "Generated from the results database by `python -m kernelforge report`. Latencies are",
        "medians over the iterations recorded with each row; the peak fraction prices the",
        f"tuned kernel against MI355X: {MI355X_CAPS.peak_hbm_gbps:.0f} GB/s HBM, "
        f"{MI355X_CAPS.peak_fp16_tflops:.1f} TFLOP/s dense fp16/bf16 MFMA, "
        f"{MI355X_CAPS.peak_fp32_tflops:.1f} TFLOP/s fp32.", "",
        "## Environment", "", *_environment(db), "",
    ]
    for warning in _warnings(rows):
        art.notes.append(warning)
        lines += [f"> **Warning:** {warning}", ""]
    present = sorted({r["operation"] for r in rows})
    for op in [o for o in (operations or present) if o in present]:
        lines += [f"## {op}", "", *_table(fastest, op), ""]
        art.tables.append(_write_csv(out / f"{op}.csv", fastest, op))
        art.figures.append(_bars(plt, fastest, op, value="median_us", ylabel="median latency (us)",
                                 title=f"{op}: latency by shape", path=out / f"{op}_latency.png"))
        has = {v for k, r in fastest.items() if k[0] == op for v in ("tflops", "gbps")
               if r.get(v) is not None}
        if op in MEMORY_BOUND_OPERATIONS:
            if "gbps" in has:
                art.figures.append(_bars(plt, fastest, op, value="gbps", ylabel="GB/s",
                                         title=f"{op}: effective bandwidth",
                                         path=out / f"{op}_bandwidth.png"))
        elif "tflops" in has:
            art.figures.append(_bars(plt, fastest, op, value="tflops", ylabel="TFLOP/s",
                                     title=f"{op}: throughput by shape",
                                     path=out / f"{op}_tflops.png"))
    heat = _heatmap(plt, rows, out / "tuning_heatmap.png")
    if heat is None:
        art.notes.append("no tuned GEMM candidates recorded, skipped tuning_heatmap.png")
    else:
        art.figures.append(heat)
    lines += ["## Files", "", *(f"- `{p.name}`" for p in (*art.tables, *art.figures)), ""]
    art.summary.write_text("\n".join(lines))
    return art
