"""Per-workload profiles of a ``bench.py`` run, from rocprofv3's output.

``bench.py --marks FILE`` launches a marker kernel before each workload (an
int8 fill of a size of its own, the only int8 fill the bench makes) and writes
FILE: the workloads in marker order, the kernel configuration dispatch picked
for each, and the source digest of the loaded library. Run that command under
rocprofv3 -- a kernel trace for durations, ``--pmc FETCH_SIZE`` and ``--pmc
WRITE_SIZE`` passes for traffic -- and this module cuts each dispatch list at
the markers, takes each workload's kernel (the library kernel it launched
most often; for the copy that calibrates the traffic counters, the copy
kernel), and writes:

* ``kernel_trace.json``: per workload the kernel name, grid and workgroup,
  its configuration, and the mean, median and minimum dispatch duration;
* ``hbm_traffic.json``: per workload FETCH_SIZE and WRITE_SIZE per dispatch
  (medians) scaled to bytes by what the same counters read for the 1 GiB copy;
* markdown tables of both, each with the commands that produced it;
* with ``--stats``, ``bench_kernel_stats.md``: rocprofv3's ``--stats`` table
  of the kernel-trace run (whole-run average per kernel), the workloads'
  kernels named.

Both JSON files carry the library's source digest and each workload's
configuration, so ``bench.py`` can refuse a profile of another build or of a
kernel dispatch no longer picks (it then reports the kernel figures as null,
with the reason).

    python -m kernelforge.profiling.bench_profiles --marks M.json --trace T.csv \\
        [--stats S.csv] [--fetch F.csv --write W.csv] [--pmc P.csv ...] \\
        [--trace-command "..."] [--traffic-command "..."] [--pmc-command "..."] --out profiles

Counter passes other than the traffic pair (``--pmc``, any counters) are
summarised per workload into ``bench_counters.json``, whose table derives the
shader clock and the matrix cores' share of busy cycles where the counters
allow.
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
from collections import Counter
from pathlib import Path

from kernelforge.profiling.rocprof import (
    Dispatch,
    allocated_vgprs,
    is_library_kernel,
    parse_counter_csv,
    parse_trace_csv,
)

#: The marker: torch's fill kernel on int8, as rocprofv3 names it demangled
#: or mangled ("a" is signed char; uint8 fills, "unsigned char" / "h", are not markers).
MARKER_NAMES = ("FillFunctor<signed char>", "FillFunctorIaE")

#: Elements of the i-th marker fill: (i + 1) * MARKER_STRIDE int8 values.
MARKER_STRIDE = 1 << 16


def is_marker(kernel: str) -> bool:
    return any(name in kernel for name in MARKER_NAMES)


def split_workloads(dispatches: list[Dispatch], names: list[str]) -> dict[str, list[Dispatch]]:
    """The dispatches between consecutive markers, keyed by workload, in launch order."""
    ordered = sorted(dispatches, key=lambda d: d.dispatch_id)
    marks = [i for i, d in enumerate(ordered) if is_marker(d.kernel)]
    if len(marks) != len(names):
        raise ValueError(f"{len(marks)} marker dispatches for {len(names)} workloads: "
                         "the profile and the marks file come from different runs")
    bounds = marks + [len(ordered)]
    return {name: ordered[bounds[i] + 1:bounds[i + 1]] for i, name in enumerate(names)}


def workload_kernel(segment: list[Dispatch], hint: str | None = None) -> list[Dispatch]:
    """The dispatches of the workload's kernel: among the library's kernels (or,
    with ``hint``, the kernels whose name contains it) the (name, grid) pair
    launched most often; the first launched wins a tie."""
    if hint is None:
        pool = [d for d in segment if is_library_kernel(d.kernel)]
    else:
        pool = [d for d in segment if hint.lower() in d.kernel.lower() and not is_marker(d.kernel)]
    if not pool:
        return []
    counts = Counter((d.kernel, d.grid) for d in pool)
    first = {}
    for d in pool:
        first.setdefault((d.kernel, d.grid), d.dispatch_id)
    key = max(counts, key=lambda k: (counts[k], -first[k]))
    return [d for d in pool if (d.kernel, d.grid) == key]


def load_marks(path: str | Path) -> dict:
    marks = json.loads(Path(path).read_text())
    if not marks.get("workloads"):
        raise ValueError(f"{path}: no workloads")
    return marks


def summarize_trace(marks: dict, trace_csv: str | Path) -> dict[str, dict]:
    """Per workload: kernel, launch shape, configuration and dispatch durations."""
    names = [w["name"] for w in marks["workloads"]]
    segments = split_workloads(parse_trace_csv(trace_csv), names)
    out = {}
    for w in marks["workloads"]:
        ds = workload_kernel(segments[w["name"]], w.get("kernel_hint"))
        if not ds:
            raise ValueError(f"workload {w['name']}: no dispatch of its kernel between its markers")
        us = [d.duration_us for d in ds]
        out[w["name"]] = {
            "kernel": ds[0].kernel, "grid": ds[0].grid, "workgroup": ds[0].workgroup,
            "vgprs": allocated_vgprs(ds[0].vgprs), "agprs": ds[0].agprs, "lds_bytes": ds[0].lds_bytes,
            "config": w.get("config"), "dispatches": len(ds),
            "mean_us": statistics.fmean(us), "median_us": statistics.median(us), "min_us": min(us),
        }
    return out


def _counter_medians(marks: dict, csv_path: str | Path, counter: str) -> dict[str, tuple[float, Dispatch, int]]:
    names = [w["name"] for w in marks["workloads"]]
    segments = split_workloads(parse_counter_csv(csv_path), names)
    out = {}
    for w in marks["workloads"]:
        ds = workload_kernel(segments[w["name"]], w.get("kernel_hint"))
        if not ds:
            raise ValueError(f"workload {w['name']}: no dispatch of its kernel in {csv_path}")
        out[w["name"]] = (statistics.median(d.counters[counter] for d in ds), ds[0], len(ds))
    return out


def summarize_traffic(marks: dict, fetch_csv: str | Path, write_csv: str | Path,
                      calibration: str = "hbm_copy_1GiB") -> dict:
    """Per workload: HBM bytes per dispatch from FETCH_SIZE and WRITE_SIZE (KiB),
    each scaled by what it reads for the calibration copy (bytes per its
    dispatch: ``copy_bytes`` read and as many written)."""
    fetch = _counter_medians(marks, fetch_csv, "FETCH_SIZE")
    write = _counter_medians(marks, write_csv, "WRITE_SIZE")
    cal = next(w for w in marks["workloads"] if w["name"] == calibration)
    copy_bytes = float(cal["copy_bytes"])
    fetch_scale = copy_bytes / (fetch[calibration][0] * 1024.0)
    write_scale = copy_bytes / (write[calibration][0] * 1024.0)
    kernels = {}
    for w in marks["workloads"]:
        f_kib, d, n = fetch[w["name"]]
        w_kib = write[w["name"]][0]
        fb, wb = f_kib * 1024.0 * fetch_scale, w_kib * 1024.0 * write_scale
        kernels[w["name"]] = {
            "kernel": d.kernel, "grid": d.grid, "config": w.get("config"), "dispatches": n,
            "fetch_kib": f_kib, "write_kib": w_kib, "fetch_bytes": fb, "write_bytes": wb,
            "traffic_bytes": fb + wb, "algorithmic_bytes": w.get("algorithmic_bytes"),
        }
    return {"calibration": {"workload": calibration, "kernel": fetch[calibration][1].kernel,
                            "copy_bytes": copy_bytes, "fetch_scale": fetch_scale,
                            "write_scale": write_scale,
                            "note": "FETCH_SIZE / WRITE_SIZE (KiB per dispatch) x 1024 x scale = bytes; "
                                    "scale = bytes the copy reads (writes) / its counter reading"},
            "kernels": kernels}


def summarize_counters(marks: dict, csv_path: str | Path) -> dict[str, dict]:
    """Per workload: the median per dispatch of every counter the pass collected."""
    names = [w["name"] for w in marks["workloads"]]
    segments = split_workloads(parse_counter_csv(csv_path), names)
    out = {}
    for w in marks["workloads"]:
        ds = workload_kernel(segments[w["name"]], w.get("kernel_hint"))
        if not ds:
            raise ValueError(f"workload {w['name']}: no dispatch of its kernel in {csv_path}")
        out[w["name"]] = {"kernel": ds[0].kernel, "grid": ds[0].grid, "config": w.get("config"),
                          "dispatches": len(ds),
                          "counters": {c: statistics.median(d.counters[c] for d in ds)
                                       for c in sorted(ds[0].counters)}}
    return out


def counters_markdown(doc: dict, durations: dict[str, float], cu_count: int = 256) -> str:
    """Counter medians per workload; with SQ_BUSY_CU_CYCLES and a kernel-trace
    duration, the shader clock; with SQ_VALU_MFMA_BUSY_CYCLES too, the share of
    SIMD busy cycles the matrix cores worked (four SIMDs per CU)."""
    names = sorted({c for e in doc["kernels"].values() for c in e["counters"]})
    head = ["workload", "dispatches", *names, "shader clock GHz", "MFMA busy / (4 x busy CU)"]
    rows = []
    for n, e in doc["kernels"].items():
        c = e["counters"]
        busy, mfma, us = c.get("SQ_BUSY_CU_CYCLES"), c.get("SQ_VALU_MFMA_BUSY_CYCLES"), durations.get(n)
        clock = f"{busy / cu_count / (us * 1e3):.2f}" if busy and us else "-"
        share = f"{100 * mfma / (4 * busy):.1f}%" if busy and mfma else "-"
        rows.append("| " + " | ".join([n, str(e["dispatches"]), *(f"{c.get(k, 0):,.0f}" for k in names),
                                       clock, share]) + " |")
    cmds = "\n".join(doc["commands"])
    return f"""# Hardware counters of every bench.py workload (rocprofv3 --pmc)

Counter passes over the same bench command, then the summary (repository root, one MI355X):

```
{cmds}
```

Library source digest: `{doc['library_digest']}`. Medians per dispatch of each workload's kernel,
found between its markers as for the kernel trace. Counters are summed over the chip: busy CU
cycles over the 256 CUs, MFMA busy cycles over the 1024 SIMDs. The shader clock is busy cycles per
CU over the median kernel-trace duration (kernel_trace.json, a separate run of the same tree).

| {" | ".join(head)} |
|{"---|" * len(head)}
""" + "\n".join(rows) + "\n"


def summarize_stats(stats_csv: str | Path, traced: dict | None = None, top: int = 12) -> list[dict]:
    """rocprofv3's ``--stats`` table (``*_kernel_stats.csv``: one row per kernel
    name over the whole run): every workload's kernel and the ``top`` kernels by
    total time, in order of total time. A kernel that is some workload's kernel
    in ``traced`` (kernel_trace.json's entries) is named by that workload, so its
    whole-run average can be set beside the per-workload median."""
    by_kernel: dict[str, list[str]] = {}
    for name, e in (traced or {}).items():
        by_kernel.setdefault(e["kernel"], []).append(name)
    rows = []
    with open(stats_csv, newline="") as handle:
        for r in csv.DictReader(handle):
            rows.append({"kernel": r["Name"], "calls": int(r["Calls"]),
                         "total_us": float(r["TotalDurationNs"]) / 1e3,
                         "average_us": float(r["AverageNs"]) / 1e3,
                         "min_us": float(r["MinNs"]) / 1e3, "max_us": float(r["MaxNs"]) / 1e3,
                         "percent": float(r["Percentage"]),
                         "workloads": by_kernel.get(r["Name"], [])})
    rows.sort(key=lambda r: -r["total_us"])
    return [r for i, r in enumerate(rows) if i < top or r["workloads"]]


def stats_markdown(rows: list[dict], commands: list[str], digest: str) -> str:
    body = "\n".join(
        f"| `{_short(r['kernel'], 70)}` | {', '.join(r['workloads']) or '-'} | {r['calls']} | "
        f"{r['average_us']:.1f} | {r['min_us']:.1f} | {r['max_us']:.1f} | {r['percent']:.1f} |"
        for r in rows)
    cmds = "\n".join(commands)
    return f"""# rocprofv3 --stats of the bench workloads run

The `--stats` table of the kernel-trace run (repository root, one MI355X), the kernels with the
most total time. Averages are over every dispatch of a kernel in the run (correctness
checks, comparisons, warm-up and timed steps), so they sit beside the per-workload medians
of `kernel_trace.json`, which count only the workload's own segment.

```
{cmds}
```

Library source digest: `{digest}`.

| kernel | workload | calls | average us | min us | max us | % of kernel time |
|---|---|---|---|---|---|---|
""" + body + "\n"


def _short(name: str, width: int = 90) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def trace_markdown(doc: dict) -> str:
    rows = [f"| {n} | `{_short(e['kernel'])}` | {e['grid']} / {e['workgroup']} | {e['vgprs']} / "
            f"{e['agprs']} | {e['lds_bytes']} | {e['dispatches']} | {e['mean_us']:.1f} | "
            f"{e['median_us']:.1f} | {e['min_us']:.1f} | `{json.dumps(e['config'], sort_keys=True)}` |"
            for n, e in doc["kernels"].items()]
    cmds = "\n".join(doc["commands"])
    return f"""# Kernel durations of every bench.py workload (rocprofv3 kernel trace)

Command (from the repository root, one MI355X, gfx950), then the summary:

```
{cmds}
```

Library source digest: `{doc['library_digest']}`. Each workload's dispatches are those of its
kernel (the library kernel it launched most often; for the copy, the copy kernel) between its
marker and the next. That counts the correctness check, the interleaved comparison with torch
where there is one, and the workload's own flushed event-timed warm-up and steps.

| workload | kernel | grid / workgroup (lanes) | VGPR / AGPR | LDS bytes | dispatches | mean us | median us | min us | configuration |
|---|---|---|---|---|---|---|---|---|---|
""" + "\n".join(rows) + "\n"


def traffic_markdown(doc: dict) -> str:
    cal = doc["calibration"]
    rows = []
    for n, e in doc["kernels"].items():
        alg = e.get("algorithmic_bytes")
        ratio = f"{e['traffic_bytes'] / alg:.2f}" if alg else "-"
        rows.append(f"| {n} | {e['dispatches']} | {e['fetch_bytes'] / 2**20:.1f} | "
                    f"{e['write_bytes'] / 2**20:.1f} | {e['traffic_bytes'] / 2**20:.1f} | "
                    f"{alg / 2**20 if alg else 0:.1f} | {ratio} |")
    cmds = "\n".join(doc["commands"])
    return f"""# HBM traffic per launch (rocprofv3 FETCH_SIZE and WRITE_SIZE)

Two counter passes over the same bench command, then the summary (repository root, one MI355X):

```
{cmds}
```

Library source digest: `{doc['library_digest']}`. Calibration: the 1 GiB device copy
(`{_short(cal['kernel'], 60)}`) reads and writes {cal['copy_bytes'] / 2**20:.0f} MiB; its counters
give fetch scale {cal['fetch_scale']:.3f} and write scale {cal['write_scale']:.3f}. The counters
see L2-to-fabric requests, so a re-read served by the 256 MiB Infinity Cache still counts.

| workload | dispatches | fetch MiB | write MiB | traffic MiB | algorithmic MiB | traffic / algorithmic |
|---|---|---|---|---|---|---|
""" + "\n".join(rows) + "\n"


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--marks", required=True, help="the file bench.py --marks wrote")
    p.add_argument("--trace", help="rocprofv3 *_kernel_trace.csv of the bench command")
    p.add_argument("--fetch", help="*_counter_collection.csv of the --pmc FETCH_SIZE pass")
    p.add_argument("--write", help="*_counter_collection.csv of the --pmc WRITE_SIZE pass")
    p.add_argument("--trace-command", action="append", default=[],
                   help="command line(s) that produced the trace, recorded in the summary")
    p.add_argument("--traffic-command", action="append", default=[],
                   help="command lines that produced the counter passes")
    p.add_argument("--pmc", action="append", default=[],
                   help="*_counter_collection.csv of any other counter pass (repeatable): "
                        "per-workload medians go to bench_counters.json")
    p.add_argument("--pmc-command", action="append", default=[],
                   help="command lines that produced the --pmc passes")
    p.add_argument("--stats", help="*_kernel_stats.csv of the kernel-trace pass (rocprofv3 --stats)")
    p.add_argument("--out", default="profiles")
    args = p.parse_args(argv)
    marks = load_marks(args.marks)
    out = Path(args.out)
    out.mkdir(parents=True, exist_ok=True)
    me = "python -m kernelforge.profiling.bench_profiles " + " ".join(
        f"--{k} {v}" for k, v in (("marks", args.marks), ("trace", args.trace), ("fetch", args.fetch),
                                  ("write", args.write)) if v)
    if args.trace:
        doc = {"commands": [*args.trace_command, me], "library_digest": marks["library_digest"],
               "note": "per-dispatch durations of each bench workload's kernel (rocprofv3 kernel trace)",
               "kernels": summarize_trace(marks, args.trace)}
        (out / "kernel_trace.json").write_text(json.dumps(doc, indent=1) + "\n")
        (out / "bench_workloads_kernel_trace.md").write_text(trace_markdown(doc))
        if args.stats:
            rows = summarize_stats(args.stats, doc["kernels"])
            (out / "bench_kernel_stats.md").write_text(
                stats_markdown(rows, [*args.trace_command, me + f" --stats {args.stats}"],
                               marks["library_digest"]))
    if args.fetch and args.write:
        doc = {"commands": [*args.traffic_command, me], "library_digest": marks["library_digest"],
               **summarize_traffic(marks, args.fetch, args.write)}
        (out / "hbm_traffic.json").write_text(json.dumps(doc, indent=1) + "\n")
        (out / "hbm_traffic_bench_workloads.md").write_text(traffic_markdown(doc))
    if args.pmc:
        merged: dict[str, dict] = {}
        for path in args.pmc:
            for name, entry in summarize_counters(marks, path).items():
                merged.setdefault(name, {**entry, "counters": {}})["counters"].update(entry["counters"])
        me_pmc = me + "".join(f" --pmc {p}" for p in args.pmc)
        doc = {"commands": [*args.pmc_command, me_pmc], "library_digest": marks["library_digest"],
               "kernels": merged}
        trace_json = out / "kernel_trace.json"
        durations = {}
        if trace_json.exists():
            traced = json.loads(trace_json.read_text())
            if traced.get("library_digest") == marks["library_digest"]:
                durations = {n: e["median_us"] for n, e in traced["kernels"].items()}
        (out / "bench_counters.json").write_text(json.dumps(doc, indent=1) + "\n")
        (out / "bench_counters_workloads.md").write_text(counters_markdown(doc, durations))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
