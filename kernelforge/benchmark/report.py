"""Reports rendered from the results database: ``summary.md``, CSV, figures.

The reference's report step (kernelforge/benchmark/report.py:263-364): every
number a reader sees comes from a row in SQLite and carries the provenance of
the run that measured it, so regenerating after a new benchmark can never
leave a stale figure behind. Only correct, timed rows are used; a fast but
wrong measurement never reaches a table or a chart.

What is specific to this build:

* implementation labels are this build's: ``torch_cpu`` (torch eager on the
  host cores), ``torch_eager`` (hipBLASLt / ATen-HIP), ``hip_default`` (the
  fixed default configuration) and ``kernelforge`` (the tuned one);
* every table row carries the MI355X roofline fraction of the best
  ``kernelforge`` measurement: GB/s over 8 TB/s for the memory-bound
  operators, TFLOP/s over the dense MFMA peak of its dtype otherwise;
* rows timed with different methods (flushed or not, HIP events or a host
  clock) are flagged rather than silently ranked together.

pandas and matplotlib are needed here and nowhere else in the package.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from math import prod
from pathlib import Path
from typing import Any

from kernelforge.db import ResultsDB
from kernelforge.runtime.env import MI355X_CAPS

#: Order of implementations in tables and legends; unknown labels follow.
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

#: The GPU timer; rows timed otherwise are host-clock measurements.
GPU_TIMER = "hip_event"


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


def _libraries() -> tuple[Any, Any]:
    try:
        import matplotlib
        import pandas
    except ImportError as exc:  # pragma: no cover - depends on the install
        raise RuntimeError("report generation needs pandas and matplotlib") from exc
    matplotlib.use("Agg")
    import matplotlib.pyplot as plt

    return pandas, plt


def _peak(operation: str, dtype: str) -> tuple[str, float]:
    if operation in MEMORY_BOUND_OPERATIONS:
        return "gbps", MI355X_CAPS.peak_hbm_gbps
    if dtype == "fp32":
        return "tflops", MI355X_CAPS.peak_fp32_tflops
    return "tflops", MI355X_CAPS.peak_fp16_tflops


def _usable(pandas: Any, db: ResultsDB):
    """Correct, timed rows, with the problem size and config keys as columns."""
    frame = pandas.DataFrame(
        [r for r in db.rows() if r["median_us"] is not None and r["correct"] != 0]
    )
    if frame.empty:
        return frame
    frame["size"] = frame["dims_json"].map(lambda s: prod(json.loads(s).values()))
    params = frame["params_json"].map(lambda s: json.loads(s) if isinstance(s, str) else {})
    for key in sorted({k for p in params for k in p}):
        frame[f"cfg_{key}"] = params.map(lambda p, k=key: p.get(k))
    return frame


def _fastest(frame):
    """Fastest row per (operation, dtype, shape, label), ordered by problem
    size (a lexicographic sort would put 512x512x512 after 2048x4096x4096)."""
    picks = frame.groupby(["operation", "dtype", "shape_key", "label"])["median_us"].idxmin()
    return frame.loc[picks].sort_values(["operation", "size", "dtype"]).copy()


def _labels(present) -> list[str]:
    present = set(present)
    known = [label for label in LABEL_ORDER if label in present]
    return known + sorted(present - set(known))


def _environment(db: ResultsDB) -> list[str]:
    runs = db.runs()
    if not runs:
        return ["No runs recorded."]
    latest = runs[-1]
    fields = (
        ("GPU", "gpu_name"),
        ("Architecture", "gpu_arch"),
        ("Compute units", "cu_count"),
        ("HIP", "hip_version"),
        ("Driver", "driver_version"),
        ("PyTorch", "torch_version"),
        ("kernelforge", "package_version"),
        ("Recorded", "timestamp"),
    )
    lines = ["| Field | Value |", "| --- | --- |"]
    lines += [f"| {title} | {latest.get(key) or '-'} |" for title, key in fields]
    return lines


def _warnings(frame) -> list[str]:
    notes = []
    if frame["flushed_l2"].nunique() > 1:
        flushed = int((frame["flushed_l2"] == 1).sum())
        notes.append(
            f"this database mixes {flushed} cache-flushed measurement(s) with "
            f"{len(frame) - flushed} unflushed; the unflushed rows report a bandwidth "
            "the kernel would not see on cold inputs, so the two are not comparable"
        )
    if frame["timer"].nunique() > 1:
        notes.append(
            f"this database mixes timers ({', '.join(sorted(frame['timer'].unique()))}); "
            f"only {GPU_TIMER} rows are GPU measurements"
        )
    return notes


def _table(best, operation: str) -> list[str]:
    labels = _labels(best["label"])
    memory_bound = operation in MEMORY_BOUND_OPERATIONS
    unit = "GB/s" if memory_bound else "TFLOP/s"
    header = ["shape", "dtype", *(f"{LABEL_TITLES.get(x, x)} (us)" for x in labels)]
    header += [f"{LABEL_TITLES[TUNED_LABEL]} {unit}", "of MI355X peak", "speedup vs eager"]
    lines = ["| " + " | ".join(header) + " |", "| " + " | ".join(["---"] * len(header)) + " |"]
    for (shape, dtype), group in best.groupby(["shape_key", "dtype"], sort=False):
        times = group.set_index("label")["median_us"]
        row = [shape, dtype] + [f"{times[x]:.1f}" if x in times else "-" for x in labels]
        column, peak = _peak(operation, dtype)
        mine = group[group["label"] == TUNED_LABEL]
        rate = mine[column].max() if not mine.empty and column in mine else None
        if rate is not None and rate == rate:
            row += [f"{rate:.1f}", f"{100.0 * rate / peak:.1f}%"]
        else:
            row += ["-", "-"]
        if TUNED_LABEL in times and "torch_eager" in times:
            row.append(f"{times['torch_eager'] / times[TUNED_LABEL]:.2f}x")
        else:
            row.append("-")
        lines.append("| " + " | ".join(row) + " |")
    return lines


def _bars(plt, best, *, value: str, ylabel: str, title: str, path: Path) -> Path:
    # One x position per (shape, dtype): the same shape measured in two dtypes
    # is two series, not one bar with two heights.
    many_dtypes = best["dtype"].nunique() > 1
    best = best.assign(
        axis_key=best["shape_key"] + (" " + best["dtype"] if many_dtypes else "")
    )
    positions = list(
        best[["axis_key", "size", "dtype"]].drop_duplicates().sort_values(["size", "dtype"])["axis_key"]
    )
    labels = _labels(best["label"])
    width = 0.8 / max(len(labels), 1)
    fig, ax = plt.subplots(figsize=(max(7.0, 1.1 * len(positions) + 2.5), 4.2))
    for i, label in enumerate(labels):
        series = best[best["label"] == label].set_index("axis_key")[value]
        heights = [float(series.get(p, float("nan"))) for p in positions]
        ax.bar([j + i * width for j in range(len(positions))], heights, width=width,
               label=LABEL_TITLES.get(label, label))
    ax.set_xticks([j + 0.4 - width / 2 for j in range(len(positions))])
    ax.set_xticklabels(positions, rotation=45, ha="right", fontsize=8)
    ax.set_ylabel(ylabel)
    ax.set_title(title)
    ax.legend(fontsize=8)
    ax.grid(axis="y", alpha=0.3)
    fig.tight_layout()
    fig.savefig(path, dpi=140)
    plt.close(fig)
    return path


def _heatmap(plt, frame, path: Path) -> Path | None:
    """Best median latency over the BLOCK_M x BLOCK_N plane of the GEMM
    (shape, dtype) with the most tuned candidates: the best each tile can do
    over the other parameters, never an average across dtypes."""
    if frame.empty or "cfg_BLOCK_M" not in frame.columns:
        return None
    tuned = frame[(frame["label"] == TUNED_LABEL) & frame["cfg_BLOCK_M"].notna()]
    if tuned.empty:
        return None
    shape, dtype = tuned.groupby(["shape_key", "dtype"])["median_us"].count().idxmax()
    chosen = tuned[(tuned["shape_key"] == shape) & (tuned["dtype"] == dtype)]
    table = chosen.pivot_table(
        index="cfg_BLOCK_M", columns="cfg_BLOCK_N", values="median_us", aggfunc="min"
    )
    if table.empty:
        return None
    fig, ax = plt.subplots(figsize=(5.6, 4.4))
    image = ax.imshow(table.values, cmap="viridis_r", aspect="auto")
    ax.set_xticks(range(len(table.columns)))
    ax.set_xticklabels([int(c) for c in table.columns])
    ax.set_yticks(range(len(table.index)))
    ax.set_yticklabels([int(i) for i in table.index])
    ax.set_xlabel("BLOCK_N")
    ax.set_ylabel("BLOCK_M")
    ax.set_title(f"Best median latency by tile ({shape} {dtype})")
    for i in range(table.shape[0]):
        for j in range(table.shape[1]):
            v = table.values[i, j]
            if v == v:
                ax.text(j, i, f"{v:.0f}", ha="center", va="center", color="white", fontsize=7)
    fig.colorbar(image, ax=ax, label="median latency (us)")
    fig.tight_layout()
    fig.savefig(path, dpi=140)
    plt.close(fig)
    return path


def generate(
    db: ResultsDB, directory: str | Path = "reports", *, operations: list[str] | None = None
) -> ReportArtifacts:
    """Write ``summary.md``, one CSV per operation and the figures into ``directory``."""
    pandas, plt = _libraries()
    out = Path(directory)
    out.mkdir(parents=True, exist_ok=True)
    artifacts = ReportArtifacts(directory=out, summary=out / "summary.md")

    frame = _usable(pandas, db)
    if frame.empty:
        artifacts.summary.write_text(
            "# kernelforge results\n\nNo correct, timed measurements in the database yet. "
            "Run `python -m kernelforge tune` or `python -m kernelforge benchmark` first.\n"
        )
        artifacts.notes.append("database contained no usable measurements")
        return artifacts

    lines = [
        "# kernelforge results",
        "",
        "Generated from the results database by `python -m kernelforge report`. Latencies are",
        "medians over the iterations recorded with each row; the peak fraction prices the",
        f"tuned kernel against MI355X: {MI355X_CAPS.peak_hbm_gbps:.0f} GB/s HBM, "
        f"{MI355X_CAPS.peak_fp16_tflops:.1f} TFLOP/s dense fp16/bf16 MFMA, "
        f"{MI355X_CAPS.peak_fp32_tflops:.1f} TFLOP/s fp32.",
        "",
        "## Environment",
        "",
        *_environment(db),
        "",
    ]
    for warning in _warnings(frame):
        artifacts.notes.append(warning)
        lines += [f"> **Warning:** {warning}", ""]

    for operation in operations or sorted(frame["operation"].unique()):
        subset = frame[frame["operation"] == operation]
        if subset.empty:
            continue
        best = _fastest(subset)
        lines += [f"## {operation}", "", *_table(best, operation), ""]
        csv = out / f"{operation}.csv"
        best.to_csv(csv, index=False)
        artifacts.tables.append(csv)
        artifacts.figures.append(
            _bars(plt, best, value="median_us", ylabel="median latency (us)",
                  title=f"{operation}: latency by shape", path=out / f"{operation}_latency.png")
        )
        if operation in MEMORY_BOUND_OPERATIONS:
            if best["gbps"].notna().any():
                artifacts.figures.append(
                    _bars(plt, best, value="gbps", ylabel="GB/s",
                          title=f"{operation}: effective bandwidth",
                          path=out / f"{operation}_bandwidth.png")
                )
        elif best["tflops"].notna().any():
            artifacts.figures.append(
                _bars(plt, best, value="tflops", ylabel="TFLOP/s",
                      title=f"{operation}: throughput by shape",
                      path=out / f"{operation}_tflops.png")
            )

    heatmap = _heatmap(plt, frame[frame["operation"] == "matmul"], out / "tuning_heatmap.png")
    if heatmap is not None:
        artifacts.figures.append(heatmap)
    else:
        artifacts.notes.append("no tuned GEMM candidates recorded, skipped tuning_heatmap.png")

    lines += ["## Files", "", *(f"- `{p.name}`" for p in (*artifacts.tables, *artifacts.figures)), ""]
    artifacts.summary.write_text("\n".join(lines))
    return artifacts
