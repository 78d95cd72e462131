"""Reading rocprofv3 output: kernel statistics and HBM traffic counters.

``read_kernel_stats`` parses ``--stats`` output (``*_kernel_stats.csv``).
``durations_by_grid`` groups a ``--kernel-trace`` (``*_kernel_trace.csv``) by
launch shape, so cells that share a kernel are timed apart.
``traffic`` combines two counter passes (``--pmc FETCH_SIZE`` and ``--pmc
WRITE_SIZE``, each a separate run: one pass cannot hold both) over the launch
sequence of ``ako_amd.benchmark.counters``. Both counters report KiB per
dispatch of traffic between the L2s and the memory fabric. Their scale
against true bytes is calibrated on the same device with the plain
elementwise kernel at the end of the sequence (1 GiB read, 1 GiB written):
``factor = expected / measured`` for each counter, applied to every cell.

    python -m ako_amd.benchmark.rocprof --fetch F.csv --write W.csv \\
        --manifest manifest.json --md profiles/<name>.md --command "..."
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import statistics
import sys
from pathlib import Path
from typing import Any

TRAFFIC_LINE = re.compile(r"^traffic (\S+) hbm_bytes_per_launch=(\d+) alg_bytes=(\d+)")


def read_kernel_stats(path: Path) -> list[dict[str, Any]]:
    """Rows of a ``*_kernel_stats.csv``: name, calls, total/avg/min/max ns, percentage."""
    rows = []
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            rows.append({
                "name": r["Name"],
                "calls": int(r["Calls"]),
                "total_ns": float(r["TotalDurationNs"]),
                "avg_ns": float(r["AverageNs"]),
                "min_ns": float(r["MinNs"]),
                "max_ns": float(r["MaxNs"]),
                "pct": float(r["Percentage"]),
            })
    return rows


def read_counters(path: Path, counter: str) -> list[dict[str, Any]]:
    """Per-dispatch ``counter`` values (KiB) in dispatch order."""
    by_dispatch: dict[int, dict[str, Any]] = {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            if r.get("Counter_Name") != counter:
                continue
            did = int(r["Dispatch_Id"])
            entry = by_dispatch.setdefault(did, {"dispatch": did, "kernel": r["Kernel_Name"], "value": 0.0})
            entry["value"] += float(r["Counter_Value"])
    return [by_dispatch[k] for k in sorted(by_dispatch)]


def _per_cell(dispatches: list[dict[str, Any]], manifest: dict[str, Any]) -> dict[str, list[float]]:
    order = manifest["dispatches"]
    tail = dispatches[-len(order):]
    if len(tail) != len(order):
        raise ValueError(f"{len(dispatches)} dispatches recorded, manifest lists {len(order)}")
    values: dict[str, list[float]] = {}
    for spec, got in zip(order, tail):
        values.setdefault(spec["cell"], []).append(got["value"] * 1024.0)
    return values


def traffic(fetch_csv: Path, write_csv: Path, manifest_path: Path) -> dict[str, Any]:
    manifest = json.loads(Path(manifest_path).read_text())
    fetch = _per_cell(read_counters(fetch_csv, "FETCH_SIZE"), manifest)
    write = _per_cell(read_counters(write_csv, "WRITE_SIZE"), manifest)
    alg = {d["cell"]: d["alg_bytes"] for d in manifest["dispatches"]}
    ref = next(c for c in alg if c.startswith("reference_"))
    expected_each = alg[ref] // 2
    f_factor = expected_each / statistics.fmean(fetch[ref])
    w_factor = expected_each / statistics.fmean(write[ref])
    kernels = {}
    for cell in alg:
        if cell == ref:
            continue
        f = statistics.fmean(fetch[cell]) * f_factor
        w = statistics.fmean(write[cell]) * w_factor
        kernels[cell] = {
            "alg_bytes": alg[cell],
            "fetch_bytes": int(f),
            "write_bytes": int(w),
            "hbm_bytes_per_launch": int(f + w),
            "traffic_over_alg": round((f + w) / alg[cell], 4),
        }
    return {
        "reference": ref,
        "fetch_factor": round(f_factor, 5),
        "write_factor": round(w_factor, 5),
        "raw_reference_fetch_kib": statistics.fmean(fetch[ref]) / 1024,
        "raw_reference_write_kib": statistics.fmean(write[ref]) / 1024,
        "kernels": kernels,
    }


def counters_by_cell(path: Path, manifest_path: Path) -> dict[str, dict[str, float]]:
    """Mean per dispatch of every counter in a ``--pmc`` collection, per cell of
    the launch manifest (instances of a counter summed within a dispatch)."""
    manifest = json.loads(Path(manifest_path).read_text())
    per_dispatch: dict[int, dict[str, float]] = {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            d = per_dispatch.setdefault(int(r["Dispatch_Id"]), {})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    order = manifest["dispatches"]
    ids = sorted(per_dispatch)[-len(order):]
    if len(ids) != len(order):
        raise ValueError(f"{len(per_dispatch)} dispatches recorded, manifest lists {len(order)}")
    sums: dict[str, dict[str, float]] = {}
    counts: dict[str, int] = {}
    for spec, did in zip(order, ids):
        cell = spec["cell"]
        acc = sums.setdefault(cell, {})
        for name, value in per_dispatch[did].items():
            acc[name] = acc.get(name, 0.0) + value
        counts[cell] = counts.get(cell, 0) + 1
    return {cell: {k: v / counts[cell] for k, v in acc.items()} for cell, acc in sums.items()}


def counters_markdown(cells: dict[str, dict[str, float]], command: str, title: str, note: str = "") -> str:
    names = sorted({n for c in cells.values() for n in c})
    lines = [f"# {title}", "", "Command:", "", "```", command, "```", ""]
    if note:
        lines += [note, ""]
    lines += ["| cell | " + " | ".join(names) + " |", "|---|" + "---:|" * len(names)]
    for cell, vals in cells.items():
        lines.append(f"| {cell} | " + " | ".join(f"{vals.get(n, 0.0):.4g}" for n in names) + " |")
    return "\n".join(lines) + "\n"


def read_kernel_trace(path: Path) -> list[tuple[str, int, int]]:
    """``(kernel name, start ns, end ns)`` rows of a ``*_kernel_trace.csv``, by start."""
    with open(path, newline="") as fh:
        rows = [(r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                for r in csv.DictReader(fh)]
    return sorted(rows, key=lambda r: r[1])


def durations_by_grid(path: Path, skip: int = 0, *, run_gap_ms: float | None = None,
                      min_calls: int = 1) -> list[dict[str, Any]]:
    """Kernel durations of a ``*_kernel_trace.csv`` grouped by (kernel, workgroup
    size, grid size): one group per launch shape, so the cells of a benchmark
    that share a kernel but not a shape come apart. ``skip`` drops each group's
    first launches (warm-up).

    A kernel compiled for dynamic shapes (a ``torch.compile(dynamic=True)``
    reduction, one program per row) can launch the same grid for rows of
    different widths. With ``run_gap_ms`` each group is further split into
    runs: a launch that starts more than ``run_gap_ms`` after the previous
    launch of its group begins a new run, so the back-to-back launches of one
    benchmarked cell stay together (``run`` numbers them in time order, from
    1). ``skip`` then applies per run, and runs left with fewer than
    ``min_calls`` launches (a lone correctness call) are dropped."""
    groups: dict[tuple[str, int, int], list[tuple[int, int]]] = {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            key = (r["Kernel_Name"], int(r["Workgroup_Size_X"]), int(r["Grid_Size_X"]))
            start = int(r["Start_Timestamp"])
            groups.setdefault(key, []).append((start, int(r["End_Timestamp"]) - start))
    out = []
    for (name, wg, grid), launches in groups.items():
        launches.sort()
        runs: list[list[int]] = [[]]
        for i, (start, ns) in enumerate(launches):
            if run_gap_ms is not None and i > 0 and start - launches[i - 1][0] > run_gap_ms * 1e6:
                runs.append([])
            runs[-1].append(ns)
        for number, ns in enumerate(runs, 1):
            ns = ns[skip:] if len(ns) > skip else ns
            if run_gap_ms is not None and len(ns) < min_calls:
                continue
            g = {"name": name, "workgroup": wg, "grid": grid, "calls": len(ns),
                 "median_us": statistics.median(ns) / 1e3, "mean_us": statistics.fmean(ns) / 1e3,
                 "min_us": min(ns) / 1e3}
            if run_gap_ms is not None:
                g["run"] = number
            out.append(g)
    return sorted(out, key=lambda g: (g["name"], g["grid"], g["workgroup"], g.get("run", 0)))


def name_matches(name: str, name_filter: str | None) -> bool:
    """True when ``name_filter`` is unset or one of its comma-separated parts
    occurs in ``name``."""
    return not name_filter or any(part and part in name for part in name_filter.split(","))


def grid_markdown(groups: list[dict[str, Any]], command: str, title: str, note: str = "",
                  name_filter: str | None = None) -> str:
    lines = [f"# {title}", "", "Command:", "", "```", command, "```", ""]
    if note:
        lines += [note, ""]
    runs = any("run" in g for g in groups)
    lines += ["| kernel | workgroup | grid (work-items) | " + ("run | " if runs else "")
              + "calls | median us | mean us | min us |",
              "|---|---:|---:|" + ("---:|" if runs else "") + "---:|---:|---:|---:|"]
    for g in groups:
        if not name_matches(g["name"], name_filter):
            continue
        name = g["name"] if len(g["name"]) <= 90 else g["name"][:87] + "..."
        run = f"{g['run']} | " if runs else ""
        lines.append(f"| `{name}` | {g['workgroup']} | {g['grid']} | {run}{g['calls']} | {g['median_us']:.2f} | "
                     f"{g['mean_us']:.2f} | {g['min_us']:.2f} |")
    return "\n".join(lines) + "\n"


def tail_breakdown(rows: list[tuple[str, int, int]], steps: int, *, tail_ms: float | None = None,
                   marker: str | None = None, library: str = "_ZN3ako") -> dict[str, Any]:
    """Kernel time per step over the last ``steps`` steps of a trace (e.g. the
    replayed decode steps that end a run). The window is either the last
    ``tail_ms`` of the trace, or -- exact -- from the end of the ``steps + 1``-th
    last launch of a kernel whose name contains ``marker`` (one launch per
    step, such as the argmax) to the end of the last one.

    Two attributions per kernel: ``us_per_step``, the sum of its recorded
    durations, and ``timeline_us_per_step``, the part of the step's span that
    ends with it: its end minus the latest end before it. On one stream the
    second partitions the span exactly, launch gaps included, while recorded
    durations of short kernels that follow a long one can start before that
    one has ended (``start_gap_us``, the median of start minus the previous
    end, is then negative) and count that overlap twice. ``library`` marks
    this library's kernels for the two totals."""
    if marker is not None:
        marks = [r for r in rows if marker in r[0]]
        if len(marks) < steps + 1:
            raise ValueError(f"{len(marks)} launches of {marker!r}, need {steps + 1}")
        begin, end = marks[-(steps + 1)][2], marks[-1][2]
        window = [r for r in rows if r[1] >= begin and r[2] <= end]
    elif tail_ms is not None:
        end = rows[-1][2]
        window = [r for r in rows if r[1] >= end - tail_ms * 1e6]
        begin = window[0][1]
    else:
        raise ValueError("give tail_ms or marker")
    per: dict[str, list[int]] = {}
    line: dict[str, int] = {}
    gaps: dict[str, list[int]] = {}
    last_end = begin
    for name, t0, t1 in window:
        per.setdefault(name, []).append(t1 - t0)
        line[name] = line.get(name, 0) + max(0, t1 - last_end)
        gaps.setdefault(name, []).append(t0 - last_end)
        last_end = max(last_end, t1)
    span_ns = end - begin
    kernels = sorted(({"name": n, "calls_per_step": len(d) / steps, "us_per_step": sum(d) / steps / 1e3,
                       "timeline_us_per_step": line[n] / steps / 1e3,
                       "start_gap_us": statistics.median(gaps[n]) / 1e3}
                      for n, d in per.items()), key=lambda k: -k["timeline_us_per_step"])
    ours = [k for k in kernels if library and library in k["name"]]
    return {"steps": steps, "span_us_per_step": span_ns / steps / 1e3,
            "busy_us_per_step": sum(k["us_per_step"] for k in kernels),
            "library_us_per_step": sum(k["us_per_step"] for k in ours),
            "library_timeline_us_per_step": sum(k["timeline_us_per_step"] for k in ours),
            "library_calls_per_step": sum(k["calls_per_step"] for k in ours),
            "kernels": kernels}


def breakdown_markdown(result: dict[str, Any], command: str, title: str, top: int = 25, note: str = "") -> str:
    lines = [f"# {title}", "", "Command:", "", "```", command, "```", ""]
    if note:
        lines += [note, ""]
    lines += [
             f"Last {result['steps']} steps of the trace: {result['span_us_per_step']:.1f} us per step, "
             f"{result['busy_us_per_step']:.1f} us of recorded kernel durations.", ""]
    if "library_timeline_us_per_step" in result:
        lines += [f"This library: {result['library_calls_per_step']:.1f} launches per step, "
                  f"{result['library_us_per_step']:.1f} us of recorded durations, "
                  f"{result['library_timeline_us_per_step']:.1f} us of the step's timeline.", "",
                  "Timeline: the kernel's end minus the latest end before it (the span is their sum, "
                  "launch gaps included). Start gap: median of its start minus that previous end; "
                  "negative when the recorded start falls inside the previous kernel.", ""]
    lines += ["| kernel | calls / step | duration us / step | timeline us / step | start gap us | share |",
              "|---|---:|---:|---:|---:|---:|"]
    for k in result["kernels"][:top]:
        name = k["name"] if len(k["name"]) <= 110 else k["name"][:107] + "..."
        tl = k.get("timeline_us_per_step", k["us_per_step"])
        share = 100.0 * tl / result["span_us_per_step"]
        gap = k.get("start_gap_us")
        gap_s = f"{gap:.2f}" if gap is not None else ""
        lines.append(f"| `{name}` | {k['calls_per_step']:.1f} | {k['us_per_step']:.1f} | {tl:.1f} | {gap_s} | "
                     f"{share:.1f}% |")
    return "\n".join(lines) + "\n"


def load_traffic_md(path: Path) -> dict[str, int]:
    """``cell -> hbm_bytes_per_launch`` from the machine-readable lines of a summary."""
    out = {}
    for line in Path(path).read_text().splitlines():
        m = TRAFFIC_LINE.match(line.strip())
        if m:
            out[m.group(1)] = int(m.group(2))
    return out


def to_markdown(result: dict[str, Any], command: str) -> str:
    lines = [
        "# HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE)",
        "",
        "Two counter passes over `python -m ako_amd.benchmark.counters`, scaled by the",
        f"plain elementwise reference `{result['reference']}` (1 GiB read + 1 GiB written):",
        f"FETCH factor {result['fetch_factor']} (raw {result['raw_reference_fetch_kib']:.0f} KiB),",
        f"WRITE factor {result['write_factor']} (raw {result['raw_reference_write_kib']:.0f} KiB).",
        "",
        "Command:",
        "",
        "```",
        command,
        "```",
        "",
        "| cell | algorithmic bytes | fetch bytes | write bytes | traffic / algorithmic |",
        "|---|---:|---:|---:|---:|",
    ]
    for cell, k in result["kernels"].items():
        lines.append(f"| {cell} | {k['alg_bytes']} | {k['fetch_bytes']} | {k['write_bytes']} | {k['traffic_over_alg']} |")
    lines += ["", "Machine-readable (read by bench.py):", "", "```"]
    for cell, k in result["kernels"].items():
        lines.append(f"traffic {cell} hbm_bytes_per_launch={k['hbm_bytes_per_launch']} alg_bytes={k['alg_bytes']}")
    lines += ["```", ""]
    return "\n".join(lines)


def launch_window(rows: list[tuple[str, int, int]], name_filter: str, first: int, count: int) -> dict[str, Any]:
    """Durations of launches ``first .. first + count - 1`` (0-based, in start
    order) of the one kernel whose name contains ``name_filter``: the launches
    a benchmark timed with its own events, to set the two clocks side by side."""
    names = {name for name, _, _ in rows if name_filter in name}
    if len(names) != 1:
        raise ValueError(f"--window {name_filter!r} matches {len(names)} kernels, expected one")
    (name,) = names
    durs = [(end - start) / 1e3 for n, start, end in rows if n == name]
    if first + count > len(durs):
        raise ValueError(f"--window asks for launches {first}..{first + count - 1} of {name}, "
                         f"the trace holds {len(durs)}")
    win = durs[first:first + count]
    return {"name": name, "first": first, "count": count, "launches_in_trace": len(durs),
            "mean_us": round(statistics.fmean(win), 2), "median_us": round(statistics.median(win), 2),
            "min_us": round(min(win), 2), "max_us": round(max(win), 2)}


def window_markdown(win: dict[str, Any], events_us: float | None) -> str:
    text = (f"Launches {win['first']}-{win['first'] + win['count'] - 1} (0-based, of {win['launches_in_trace']}) "
            f"of `{win['name'][:90]}...`, the {win['count']} that bench.py timed with an event pair each "
            f"(`roofline.event_launches`): mean {win['mean_us']:.2f} us, median {win['median_us']:.2f} us, "
            f"min {win['min_us']:.2f} us, max {win['max_us']:.2f} us by kernel duration")
    if events_us is not None:
        text += (f"; the same launches by the events of the same run: mean {events_us:.2f} us "
                 f"(`roofline.mean_launch_us`), {100 * (events_us / win['mean_us'] - 1):+.1f}%")
    return text + ".\n"


def stats_markdown(rows: list[dict[str, Any]], command: str, title: str, top: int = 40) -> str:
    lines = [f"# {title}", "", "Command:", "", "```", command, "```", "",
             "| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---:|---:|---:|---:|---:|"]
    for r in sorted(rows, key=lambda r: -r["total_ns"])[:top]:
        name = r["name"] if len(r["name"]) <= 110 else r["name"][:107] + "..."
        lines.append(f"| `{name}` | {r['calls']} | {r['avg_ns'] / 1e3:.2f} | {r['min_ns'] / 1e3:.2f} | "
                     f"{r['max_ns'] / 1e3:.2f} | {r['pct']:.2f} |")
    return "\n".join(lines) + "\n"


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--fetch", type=Path)
    ap.add_argument("--write", type=Path)
    ap.add_argument("--manifest", type=Path)
    ap.add_argument("--stats", type=Path, help="a *_kernel_stats.csv to summarise instead")
    ap.add_argument("--trace", type=Path, help="a *_kernel_trace.csv: per-step breakdown of its tail")
    ap.add_argument("--pmc", type=Path, help="a *_counter_collection.csv: every counter per cell (with --manifest)")
    ap.add_argument("--note", default="", help="with --pmc, --by-grid or --trace: a sentence placed above the table")
    ap.add_argument("--by-grid", action="store_true",
                    help="with --trace: durations per (kernel, workgroup, grid) instead of a tail breakdown")
    ap.add_argument("--skip", type=int, default=0, help="with --by-grid: warm-up launches dropped per group")
    ap.add_argument("--filter", default=None,
                    help="with --by-grid: only kernels whose name contains this (or one of several, comma-separated)")
    ap.add_argument("--run-gap-ms", type=float, default=None,
                    help="with --by-grid: split each group into runs at start gaps above this many ms")
    ap.add_argument("--min-calls", type=int, default=1,
                    help="with --run-gap-ms: drop runs with fewer launches (after --skip)")
    ap.add_argument("--tail-ms", type=float, default=None, help="with --trace: window at the end of the run")
    ap.add_argument("--steps", type=int, default=None, help="with --trace: steps inside the window")
    ap.add_argument("--marker", default=None, help="with --trace: a kernel launched once per step")
    ap.add_argument("--title", default="rocprofv3 kernel statistics")
    ap.add_argument("--command", default="")
    ap.add_argument("--md", type=Path, required=True)
    ap.add_argument("--json", type=Path, help="also write the figures as JSON (e.g. next to a BenchmarkReport)")
    ap.add_argument("--window", default=None, metavar="SUBSTR:FIRST:COUNT",
                    help="with --stats and --trace: kernel durations of launches FIRST..FIRST+COUNT-1 of "
                         "the kernel whose name contains SUBSTR")
    ap.add_argument("--bench-json", type=Path, default=None,
                    help="with --window: the bench.py line of the same run, for its event timing")
    args = ap.parse_args(argv)
    if args.pmc:
        cells = counters_by_cell(args.pmc, args.manifest)
        args.md.write_text(counters_markdown(cells, args.command, args.title, args.note))
        record: dict[str, Any] = {"kind": "counters_by_cell", "title": args.title, "cells": cells}
    elif args.trace and args.by_grid:
        groups = durations_by_grid(args.trace, args.skip, run_gap_ms=args.run_gap_ms, min_calls=args.min_calls)
        groups = [g for g in groups if name_matches(g["name"], args.filter)]
        args.md.write_text(grid_markdown(groups, args.command, args.title, args.note))
        record = {"kind": "durations_by_grid", "title": args.title, "groups": groups}
    elif args.trace and not args.stats:
        result = tail_breakdown(read_kernel_trace(args.trace), args.steps, tail_ms=args.tail_ms,
                                marker=args.marker)
        args.md.write_text(breakdown_markdown(result, args.command, args.title, note=args.note))
        record = {"kind": "trace_tail_breakdown", "title": args.title, **result}
    elif args.stats:
        rows = read_kernel_stats(args.stats)
        text = stats_markdown(rows, args.command, args.title)
        record = {"kind": "kernel_stats", "title": args.title, "kernels": rows}
        if args.window:
            if not args.trace:
                ap.error("--window needs --trace")
            substr, first, count = args.window.rsplit(":", 2)
            win = launch_window(read_kernel_trace(args.trace), substr, int(first), int(count))
            events_us = None
            if args.bench_json:
                line = args.bench_json.read_text().strip().splitlines()[-1]
                events_us = json.loads(line)["roofline"]["mean_launch_us"]
            text += "\n" + window_markdown(win, events_us)
            record["window"] = {**win, "events_mean_us": events_us}
        args.md.write_text(text)
    else:
        result = traffic(args.fetch, args.write, args.manifest)
        args.md.write_text(to_markdown(result, args.command))
        record = {"kind": "hbm_traffic", **result}
    if args.json:
        args.json.parent.mkdir(parents=True, exist_ok=True)
        args.json.write_text(json.dumps({**record, "command": args.command}, indent=2) + "\n")
    print(args.md.read_text())
    return 0


if __name__ == "__main__":
    sys.exit(main())
