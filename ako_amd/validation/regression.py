"""Latency-regression diff between two benchmark reports.

Follows ``ako/validation/regression.py:14-26``: rows of ``comparisons[]`` are
matched on ``(shape, selected_kernel)`` (plus ``dtype`` when both rows carry
it, so fp16 and bf16 cells of one shape are not conflated) and a candidate
latency that grew by more than ``rtol`` is reported.
"""

from __future__ import annotations

import json
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
