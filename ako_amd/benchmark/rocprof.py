"""Reading rocprofv3 output: kernel statistics and HBM traffic counters.

``read_kernel_stats`` parses ``--stats`` output (``*_kernel_stats.csv``).
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
    ap.add_argument("--title", default="rocprofv3 kernel statistics")
    ap.add_argument("--command", default="")
    ap.add_argument("--md", type=Path, required=True)
    ap.add_argument("--json", type=Path, help="also write the figures as JSON (e.g. next to a BenchmarkReport)")
    args = ap.parse_args(argv)
    if args.stats:
        rows = read_kernel_stats(args.stats)
        args.md.write_text(stats_markdown(rows, args.command, args.title))
        record: dict[str, Any] = {"kind": "kernel_stats", "title": args.title, "kernels": rows}
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
