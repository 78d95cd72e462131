"""Benchmark reports: raw ``results[]`` rows and ``comparisons[]`` rows.

The JSON layout is the reference's (``ako/benchmark/report.py:15-87``) so the
regression diff and any downstream tooling read both. Comparison rows may
carry extra MI355X columns (``alg_bytes``, ``gbps``, ``pct_hbm_peak``,
``err_ulps``, ``fetch_bytes``, ``write_bytes``) through ``**extra``.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

from ako_amd.benchmark.bench_op import BenchResult
from ako_amd.dispatcher.hardware import DeviceInfo


@dataclass
class BenchmarkReport:
    operation: str
    device: DeviceInfo
    results: list[dict[str, Any]] = field(default_factory=list)
    comparisons: list[dict[str, Any]] = field(default_factory=list)
    created_at: str = field(default_factory=lambda: datetime.now(timezone.utc).isoformat())
    #: Optional rocprofv3 counter figures (``ako_amd.benchmark.rocprof.traffic``)
    #: stored beside the timing rows; absent from the JSON when unset, so
    #: reports keep the reference's layout.
    counters: dict[str, Any] | None = None

    def add_result(self, result: BenchResult, **extra: Any) -> None:
        self.results.append({**result.to_dict(), **extra})

    def add_comparison(
        self,
        *,
        shape: list[int],
        baseline_ms: float,
        candidate_ms: float,
        max_error: float,
        selected_kernel: str,
        dtype: str | None = None,
        baseline_kernel: str = "rmsnorm_ref",
        best_baseline_ms: float | None = None,
        best_baseline_kernel: str | None = None,
        **extra: Any,
    ) -> None:
        """One candidate against the unfused reference and the best baseline."""
        row: dict[str, Any] = {
            "shape": shape,
            "baseline_ms": round(baseline_ms, 4),
            "baseline_kernel": baseline_kernel,
            "candidate_ms": round(candidate_ms, 4),
            "speedup": round(baseline_ms / candidate_ms, 3) if candidate_ms > 0 else 0.0,
            "max_error": max_error,
            "selected_kernel": selected_kernel,
        }
        if dtype is not None:
            row["dtype"] = dtype
        if best_baseline_ms is not None:
            row["best_baseline_ms"] = round(best_baseline_ms, 4)
            row["best_baseline_kernel"] = best_baseline_kernel
            row["speedup_vs_best_baseline"] = (
                round(best_baseline_ms / candidate_ms, 3) if candidate_ms > 0 else 0.0
            )
        row.update(extra)
        self.comparisons.append(row)

    def attach_counters(self, traffic_result: dict[str, Any]) -> None:
        """Keep counter-measured HBM traffic next to the timings, and add
        ``fetch_bytes`` / ``write_bytes`` / ``traffic_over_alg`` to every
        comparison row whose ``cell`` names a measured kernel."""
        self.counters = traffic_result
        kernels = traffic_result.get("kernels", {})
        for row in self.comparisons:
            k = kernels.get(row.get("cell"))
            if k is not None:
                row.update(fetch_bytes=k["fetch_bytes"], write_bytes=k["write_bytes"],
                           traffic_over_alg=k["traffic_over_alg"])

    def to_dict(self) -> dict[str, Any]:
        out = {
            "operation": self.operation,
            "gpu": self.device.device_name,
            "device": self.device.to_dict(),
            "created_at": self.created_at,
            "results": self.results,
            "comparisons": self.comparisons,
        }
        if self.counters is not None:
            out["counters"] = self.counters
        return out


def save_report(report: BenchmarkReport, path: str | Path) -> Path:
    out = Path(path)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(report.to_dict(), indent=2))
    return out
