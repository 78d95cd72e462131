"""Selection sweep over the BASELINE.json grid: which kernel wins each cell.

For every cell of configs[1]-[3] (RMSNorm and residual RMSNorm, RoPE q and
k, SwiGLU; prefill and decode sizes) a fresh ``KernelSelector`` runs the
reference's Algorithm 1 on the GPU: the unfused reference, the PyTorch
baselines and the HIP candidate are gated and timed (wall p50 per call,
the reference's selection criterion), and the decision is recorded. The
output rows follow the reference's ``comparisons[]`` format (what
``ako/benchmark/rmsnorm_bench.py`` and ``rope_bench.py`` wrote), one report
per operation, plus a summary with the HIP win rate.

    python -m ako_amd.benchmark.sweep --out out/selection [--ops rmsnorm,rope]
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from pathlib import Path
from typing import Any, Callable, Iterator

import torch

from ako_amd.benchmark.report import BenchmarkReport, save_report
from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.hardware import get_device_info
from ako_amd.dispatcher.registry import KernelRegistry
from ako_amd.dispatcher.selector import KernelSelector
from ako_amd.ops._registry import register_all
from ako_amd.ops.rope_ref import build_rope_tables

RMS_HIDDEN = (4096, 8192, 16384)
RMS_ROWS = (1, 32, 16384)
ROPE_BS = ((1, 1), (64, 1), (4, 2048))
SWIGLU_M = (1, 16, 256, 4096, 16384)
HALF = (torch.float16, torch.bfloat16)


def _randn(shape, dtype, seed, device, scale=1.0, shift=0.0) -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=device) * scale + shift).to(dtype)


def cells(ops: set[str], device: torch.device) -> Iterator[tuple[str, list[int], torch.dtype, tuple, dict]]:
    """``(op, shape, dtype, tensors, select kwargs)`` for every grid cell."""
    for dtype in HALF:
        for h in RMS_HIDDEN:
            for rows in RMS_ROWS:
                x = _randn((rows, h), dtype, 0, device)
                w = _randn((h,), dtype, 1, device, 0.1, 1.0)
                if "rmsnorm" in ops:
                    yield "rmsnorm", [rows, h], dtype, (x, w), {}
                if "rmsnorm_residual" in ops:
                    r = _randn((rows, h), dtype, 2, device)
                    yield "rmsnorm_residual", [rows, h], dtype, (x, r, w), {}
    if "rope" in ops or "rope_qk" in ops:
        for dtype in HALF:
            for b, s in ROPE_BS:
                cos, sin = build_rope_tables(s, 128, device=device)
                cos, sin = cos.to(dtype), sin.to(dtype)
                q = _randn((b, s, 32, 128), dtype, 3, device)
                k = _randn((b, s, 8, 128), dtype, 6, device)
                if "rope" in ops:
                    for x in (q, k):
                        yield "rope", list(x.shape), dtype, (x, cos, sin), {
                            "extra_key": "neox", "call_kwargs": {"style": "neox"}}
                if "rope_qk" in ops:
                    yield "rope_qk", [b, s, 32 + 8, 128], dtype, (q, k, cos, sin), {
                        "extra_key": "neox", "call_kwargs": {"style": "neox"}}
    if "swiglu" in ops:
        for m in SWIGLU_M:
            g = _randn((m, 14336), torch.bfloat16, 4, device)
            u = _randn((m, 14336), torch.bfloat16, 5, device)
            yield "swiglu", [m, 14336], torch.bfloat16, (g, u), {}


def cell_name(op: str, shape: list[int], dtype: torch.dtype) -> str:
    """The cell's name as the counter runs (``ako_amd.benchmark.counters``)
    and ``bench.py`` spell it, so counter figures can be attached to rows."""
    tag = {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}[dtype]
    if op in ("rmsnorm", "rmsnorm_residual"):
        return f"{op}_{tag}_{shape[0]}x{shape[1]}"
    if op == "rope":
        which = "q" if shape[2] == 32 else "k"
        return f"rope_{which}_{tag}_{shape[0]}x{shape[1]}x{shape[2]}x{shape[3]}"
    if op == "rope_qk":
        return f"rope_qk_{tag}_{shape[0]}x{shape[1]}"
    return f"{op}_{tag}_{'x'.join(map(str, shape))}"


def is_decode(op: str, shape: list[int]) -> bool:
    """Decode-sized cells: at most 32 rows, one token per sequence, M <= 16."""
    if op in ("rmsnorm", "rmsnorm_residual"):
        return shape[0] <= 32
    if op in ("rope", "rope_qk"):
        return shape[1] == 1
    return shape[0] <= 16


def run(out_dir: Path, ops: set[str], *, warmup: int = 5, repeats: int = 20,
        counters: dict[str, Any] | None = None,
        keep: Callable[[str, list[int], torch.dtype], bool] | None = None,
        quiet: bool = False) -> dict[str, Any]:
    """Select every cell (or those ``keep(op, shape, dtype)`` accepts); write
    one report per op and a summary, and return the summary."""
    device = torch.device("cuda", torch.cuda.current_device())
    info = get_device_info(device)
    registry = register_all(KernelRegistry())
    reports: dict[str, BenchmarkReport] = {}
    wins = total = decode_total = decode_wins = 0
    others: list[dict[str, Any]] = []
    leads: dict[str, list[float]] = {}
    worst_ulps: dict[str, float] = {}
    for op, shape, dtype, tensors, kw in cells(ops, device):
        if keep is not None and not keep(op, shape, dtype):
            continue
        selector = KernelSelector(registry=registry, cache=KernelCache(path=out_dir / "sweep_cache.json"),
                                  auto_tune=True, warmup=warmup, repeats=repeats)
        result = selector.select_entry(op, *tensors, **kw)
        lat = dict(result.latencies_ms)
        hip_name = f"{op}_hip"
        hip_report = next((r for r in result.ulp_reports if r["kernel"] == hip_name), None)
        report = reports.setdefault(op, BenchmarkReport(operation=op, device=info))
        report.add_comparison(
            shape=shape,
            dtype=str(dtype).replace("torch.", ""),
            cell=cell_name(op, shape, dtype),
            baseline_ms=result.baseline_ms or 0.0,
            baseline_kernel=f"{op}_ref",
            candidate_ms=lat.get(hip_name, float("nan")),
            max_error=hip_report["max_error"] if hip_report else None,
            selected_kernel=result.entry.kernel_name,
            best_baseline_ms=result.best_baseline_ms,
            best_baseline_kernel=result.best_baseline_kernel,
            err_ulps=hip_report["err_ulps"] if hip_report else None,
            gate_passed=hip_report["passed"] if hip_report else None,
            latencies_ms={k: round(v, 5) for k, v in lat.items()},
            rejected=list(result.rejected),
        )
        if hip_report is not None and hip_report.get("err_ulps") is not None:
            worst_ulps[op] = max(worst_ulps.get(op, 0.0), float(hip_report["err_ulps"]))
        hip_won = result.entry.backend == "hip"
        total += 1
        wins += int(hip_won)
        if is_decode(op, shape):
            decode_total += 1
            decode_wins += int(hip_won)
        if not hip_won:
            others.append({"cell": cell_name(op, shape, dtype), "selected": result.entry.kernel_name,
                           "latencies_us": {k: round(v * 1e3, 2) for k, v in lat.items()}})
        if result.speedup_vs_best_baseline:
            phase = "decode" if is_decode(op, shape) else "prefill"
            leads.setdefault(f"{op}_{phase}", []).append(result.speedup_vs_best_baseline)
        if not quiet:
            print(f"[sweep] {op:17s} {str(shape):22s} {str(dtype)[6:]:9s} -> {result.entry.kernel_name:22s} "
                  + " ".join(f"{k}={v * 1e3:.1f}us" for k, v in lat.items()), flush=True)
        del tensors
    out_dir.mkdir(parents=True, exist_ok=True)
    for op, report in reports.items():
        if counters is not None:
            report.attach_counters(counters)
        save_report(report, out_dir / f"selection_{op}.json")
    summary = {"cells": total, "hip_selected": wins, "hip_win_rate": round(wins / total, 4) if total else None,
               "decode_cells": decode_total, "decode_hip_selected": decode_wins,
               # The reference campaign's headline numbers (scripts/run_campaign.py:287-337):
               # the selected kernel's median lead over the fastest baseline, per op and phase.
               "median_lead_vs_best_baseline": {k: round(statistics.median(v), 3) for k, v in sorted(leads.items())},
               # The HIP candidate's largest error over each op's cells, in ulps
               # of the reference output's largest magnitude (the gate's report).
               "max_err_ulps": {k: round(v, 3) for k, v in sorted(worst_ulps.items())},
               "not_hip": others, "gpu": info.device_name, "cache_key": info.cache_key}
    (out_dir / "selection_summary.json").write_text(json.dumps(summary, indent=2))
    return summary


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", type=Path, required=True)
    ap.add_argument("--ops", default="rmsnorm,rmsnorm_residual,rope,rope_qk,swiglu")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--repeats", type=int, default=20)
    ap.add_argument("--counters", type=Path, default=None,
                    help="HBM-traffic JSON from `python -m ako_amd.benchmark.rocprof ... --json` to attach")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("the selection sweep needs a GPU", file=sys.stderr)
        return 1
    counters = json.loads(args.counters.read_text()) if args.counters else None
    summary = run(args.out, set(args.ops.split(",")), warmup=args.warmup, repeats=args.repeats,
                  counters=counters)
    print(json.dumps(summary), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
