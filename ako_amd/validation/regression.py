"""Regression diffs between two runs.

``compare_reports`` follows ``ako/validation/regression.py:14-26``: rows of
``comparisons[]`` are matched on ``(shape, selected_kernel)`` (plus ``dtype``
when both rows carry it, so fp16 and bf16 cells of one shape are not
conflated) and a candidate latency that grew by more than ``rtol`` is
reported. ``compare_bench_lines`` does the same for two ``bench.py`` JSON
lines: the step throughput, every per-kernel and extra cell's bandwidth (or
graph-replay time for decode-size cells) and the decoder timings.

    python -m ako_amd.validation.regression CURRENT.json PREVIOUS.json [--rtol 0.1]
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path
from typing import Any


def load_baseline(path: str | Path) -> dict[str, Any]:
    return json.loads(Path(path).read_text())


def _row_key(row: dict[str, Any]) -> tuple[Any, ...]:
    return (tuple(row["shape"]), row["selected_kernel"], row.get("dtype"))


def compare_reports(
    current: dict[str, Any], baseline: dict[str, Any], *, rtol: float = 0.1
) -> list[str]:
    """Human-readable warnings for every comparison row that got slower."""
    previous = {_row_key(r): r for r in baseline.get("comparisons", [])}
    warnings: list[str] = []
    for row in current.get("comparisons", []):
        old = previous.get(_row_key(row))
        if old is None:
            continue
        before, now = old["candidate_ms"], row["candidate_ms"]
        if before > 0 and (now - before) / before > rtol:
            warnings.append(f"Regression on {_row_key(row)}: {before:.3f}ms -> {now:.3f}ms")
    return warnings


def _last_json_line(text: str) -> dict[str, Any]:
    """A whole JSON document, or else the last line of a log that is one
    (``bench.py`` prints its record as the last line of its output)."""
    try:
        return json.loads(text)
    except json.JSONDecodeError:
        lines = [ln for ln in text.strip().splitlines() if ln.strip().startswith("{")]
        return json.loads(lines[-1])


def compare_bench_lines(
    current: dict[str, Any], baseline: dict[str, Any], *, rtol: float = 0.05
) -> list[str]:
    """Warnings for every figure of a ``bench.py`` line that got worse by more
    than ``rtol``: lower GB/s, or higher decode-cell and decoder times."""
    warnings: list[str] = []

    def worse(label: str, before: float | None, now: float | None, higher_is_better: bool) -> None:
        if before is None or now is None or before <= 0:
            return
        change = (before - now) / before if higher_is_better else (now - before) / before
        if change > rtol:
            warnings.append(f"Regression on {label}: {before:g} -> {now:g}")

    if current.get("metric") != baseline.get("metric"):
        return [f"Different metrics: {current.get('metric')!r} vs {baseline.get('metric')!r}"]
    worse("value", baseline.get("value"), current.get("value"), bool(current.get("higher_is_better", True)))
    for table in ("per_kernel", "extras"):
        previous = {row["name"]: row for row in baseline.get(table) or []}
        for row in current.get(table) or []:
            old = previous.get(row["name"])
            if old is None:
                continue
            if "graph_us" in row and "graph_us" in old:
                worse(f"{row['name']} graph_us", old["graph_us"], row["graph_us"], False)
            else:
                worse(f"{row['name']} GB/s", old.get("gbps"), row.get("gbps"), True)
    for backend in ("ako",):
        old = (baseline.get("decoder") or {}).get(backend) or {}
        new = (current.get("decoder") or {}).get(backend) or {}
        for key in ("prefill_ms", "decode_ms_per_step", "graphed_decode_ms_per_step"):
            worse(f"decoder {backend} {key}", old.get(key), new.get(key), False)
    return warnings


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("current", type=Path)
    ap.add_argument("baseline", type=Path)
    ap.add_argument("--rtol", type=float, default=None)
    args = ap.parse_args(argv)
    cur = _last_json_line(args.current.read_text())
    base = _last_json_line(args.baseline.read_text())
    if "comparisons" in cur:
        warnings = compare_reports(cur, base, rtol=args.rtol if args.rtol is not None else 0.1)
    else:
        warnings = compare_bench_lines(cur, base, rtol=args.rtol if args.rtol is not None else 0.05)
    for w in warnings:
        print(w)
    print(f"{len(warnings)} regression(s)")
    return 1 if warnings else 0


if __name__ == "__main__":
    sys.exit(main())
