"""In-process kernel-time breakdown with ``torch.profiler`` (reference
``ako/benchmark/profiler.py:11-26`` wraps the same profiler).

``rocprofv3`` (``ako_amd.benchmark.rocprof``) is the instrument of record for
kernel durations and counters, but it needs its own process. For a quick
answer inside a running program, "where does a decode step's device time go,
and how much of it is this library's kernels", ``profile_cuda`` records a
region and ``kernel_table`` folds the recorded device kernels by name:

    with profile_cuda() as prof:
        step()
    rows = kernel_table(prof)
    print(library_share(rows))

Kernels of this library are recognised by their ``ako`` namespace, whether
the profiler reports the demangled name (``ako::rmsnorm_reg<...>``) or the
mangled symbol (``_ZN3ako11rmsnorm_reg...``).
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any, Iterator

import torch

LIBRARY_MARKERS = ("ako::", "_ZN3ako")


def is_library_kernel(name: str, markers: tuple[str, ...] = LIBRARY_MARKERS) -> bool:
    return any(m in name for m in markers)


@contextmanager
def profile_cuda(activities: list[Any] | None = None) -> Iterator[torch.profiler.profile]:
    """Profile the enclosed region (host ops, and device kernels on a GPU)."""
    if activities is None:
        activities = [torch.profiler.ProfilerActivity.CPU]
        if torch.cuda.is_available():
            activities.append(torch.profiler.ProfilerActivity.CUDA)
    with torch.profiler.profile(activities=activities, record_shapes=True) as prof:
        yield prof


def _device_us(event: Any) -> float:
    for attr in ("self_device_time_total", "self_cuda_time_total"):
        value = getattr(event, attr, None)
        if value:
            return float(value)
    return 0.0


def _is_host_event(event: Any) -> bool:
    kind = getattr(event, "device_type", None)
    return kind is not None and str(kind).rsplit(".", 1)[-1] == "CPU"


def kernel_table(prof: torch.profiler.profile, *, device: bool | None = None) -> list[dict[str, Any]]:
    """Rows ``{name, calls, total_us, avg_us, share}`` sorted by total time.

    ``device`` True folds device kernel time (a GPU run), False host op time
    (a CPU-only run); by default device time when any was recorded. ``share``
    is each row's fraction of the table's total.
    """
    events = list(prof.key_averages())
    if device is None:
        device = any(_device_us(e) > 0 for e in events)
    rows = []
    for e in events:
        # Device rows are kernels only: a host op (aten::mm) also reports the
        # device time of the kernels it launched, which would count them twice.
        if device and _is_host_event(e):
            continue
        total = _device_us(e) if device else float(getattr(e, "self_cpu_time_total", 0.0) or 0.0)
        if total <= 0:
            continue
        rows.append({"name": e.key, "calls": int(e.count), "total_us": total,
                     "avg_us": total / max(int(e.count), 1)})
    grand = sum(r["total_us"] for r in rows) or 1.0
    for r in rows:
        r["share"] = r["total_us"] / grand
    rows.sort(key=lambda r: r["total_us"], reverse=True)
    return rows


def library_share(rows: list[dict[str, Any]], markers: tuple[str, ...] = LIBRARY_MARKERS) -> dict[str, Any]:
    """Time in this library's kernels against everything else in ``rows``."""
    ours = [r for r in rows if is_library_kernel(r["name"], markers)]
    total = sum(r["total_us"] for r in rows)
    mine = sum(r["total_us"] for r in ours)
    return {"library_us": mine, "total_us": total, "share": mine / total if total else 0.0,
            "library_kernels": sorted({r["name"] for r in ours}),
            "library_calls": sum(r["calls"] for r in ours)}


def table_markdown(rows: list[dict[str, Any]], *, top: int = 20, per: int = 1) -> str:
    """A markdown table of the ``top`` rows, times divided by ``per`` (e.g. steps)."""
    lines = ["| kernel | calls | total us | share |", "|---|---:|---:|---:|"]
    for r in rows[:top]:
        lines.append(f"| `{r['name'][:90]}` | {r['calls'] / per:g} | {r['total_us'] / per:.1f} | "
                     f"{100 * r['share']:.1f}% |")
    return "\n".join(lines)
