"""The one JSON line ``bench.py`` prints, and the per-cell report beside it.

The line carries the headline figures only (value, roofline, CPU baseline,
selection counts, the decoder summary, the RoPE prefill cells and each op's
lowest prefill share of peak) and must stay well under ``LINE_LIMIT`` bytes,
so that a reader that keeps only the tail of the output still holds all of
it. Every timed cell goes to a report file instead, in the reference's
report layout (``operation``/``gpu``/``device``/``created_at``/``results``/
``comparisons``, ``ako/benchmark/report.py:15-87``): one ``results`` row per
cell, and the selection's ``comparisons`` rows.
"""

from __future__ import annotations

import json
import math
import re
from datetime import datetime, timezone
from typing import Any

#: Hard ceiling on the printed line, bytes.
LINE_LIMIT = 8192

_CELL = re.compile(r"^(?P<op>[a-z_]+?)_(?P<dt>fp16|bf16|fp32)_(?P<shape>\d+(?:x\d+)*)(?:_(?P<rest>.+))?$")
_DTYPES = {"fp16": "float16", "bf16": "bfloat16", "fp32": "float32"}

#: Cells whose share of peak is held to the >= 75% prefill target, by op:
#: RMSNorm rows = 16384, RoPE (4, 2048) (also with the KV-cache write, as the
#: decoder calls it), SwiGLU M in {4096, 16384}.
PREFILL = {
    "rmsnorm": re.compile(r"^rmsnorm_(fp16|bf16)_16384x\d+$"),
    "rmsnorm_residual": re.compile(r"^rmsnorm_residual_(fp16|bf16)_16384x\d+$"),
    "rope_qk": re.compile(r"^rope_qk_(fp16|bf16)_4x2048$"),
    "rope_qk_cache": re.compile(r"^rope_qk_cache_(fp16|bf16)_4x2048_q32_kv8$"),
    "rope_q": re.compile(r"^rope_q_(fp16|bf16)_4x2048x32x128$"),
    "swiglu": re.compile(r"^swiglu_bf16_(4096|16384)x14336$"),
}


def parse_cell(name: str) -> dict[str, Any]:
    """``{"op", "dtype", "shape", "variant"}`` from a cell name such as
    ``rmsnorm_residual_fp16_16384x8192`` or ``rope_q_bf16_4x2048x32x128``."""
    m = _CELL.match(name)
    if m is None:
        return {"op": name, "dtype": None, "shape": [], "variant": None}
    return {"op": m["op"], "dtype": _DTYPES[m["dt"]], "shape": [int(v) for v in m["shape"].split("x")],
            "variant": m["rest"]}


def _b2b_pct(row: dict[str, Any]) -> float:
    """A row's share of peak timed back to back: the step's cells carry it
    under ``back_to_back`` (their top-level figure is per launch); the extras
    are timed back to back at the top level."""
    return (row.get("back_to_back") or {}).get("pct_hbm_peak", row["pct_hbm_peak"])


def _launch_pct(row: dict[str, Any]) -> float | None:
    """A row's share of peak per launch, from events bound to each launch
    (the kernel's own duration): the step's cells at the top level, the
    extras under ``per_launch`` (None when they have none)."""
    if "back_to_back" in row:
        return row["pct_hbm_peak"]
    return (row.get("per_launch") or {}).get("pct_hbm_peak")


def prefill_floor(rows: list[dict[str, Any]]) -> dict[str, dict[str, Any]]:
    """Per op, the prefill cell with the lowest share of peak timed back to
    back (and how many prefill cells there were), and the lowest per-launch
    figure where the cells have one, from rows carrying ``name``/
    ``pct_hbm_peak`` (``back_to_back`` for the step's cells, ``per_launch``
    for the extras)."""
    out: dict[str, dict[str, Any]] = {}
    for op, pat in PREFILL.items():
        hits = [r for r in rows if pat.match(r["name"])]
        if hits:
            low = min(hits, key=_b2b_pct)
            out[op] = {"min_pct": _b2b_pct(low), "cell": low["name"], "cells": len(hits)}
            timed = [(p, r["name"]) for r in hits if (p := _launch_pct(r)) is not None]
            if len(timed) == len(hits):
                pct, name = min(timed)
                out[op]["min_per_launch_pct"] = pct
                out[op]["per_launch_cell"] = name
    return out


def selection_summary(sel: dict[str, Any] | None) -> dict[str, Any] | None:
    if sel is None:
        return None
    keep = ("cells", "hip_selected", "win_rate", "decode_cells", "decode_hip_selected", "max_err_ulps")
    out = {k: sel[k] for k in keep if k in sel}
    out["not_hip"] = len(sel.get("not_hip", []))
    return out


def decoder_summary(dec: dict[str, Any] | None) -> dict[str, Any] | None:
    """configs[4] as one flat level of figures."""
    if dec is None:
        return None
    out: dict[str, Any] = {}
    for backend in ("torch", "ako"):
        r = dec.get(backend, {})
        for k in ("prefill_ms", "decode_ms", "decode_ms_per_step", "graphed_decode_ms_per_step"):
            if k in r:
                out[f"{backend}_{k}"] = r[k]
    for k in ("prefill_speedup", "decode_speedup", "graphed_decode_speedup", "greedy_tokens_identical"):
        if k in dec:
            out[k] = dec[k]
    step = dec.get("ako", {}).get("graphed_step_breakdown") or {}
    if step.get("recorded"):
        # Recorded kernel durations under the profiler: each includes the
        # launch's dispatch behind the kernel before it.
        out["graphed_step_device_recorded_us"] = step["device_us_per_step"]
        out["graphed_step_library_recorded_us"] = step["library_us_per_step"]
    return out


def compact_line(full: dict[str, Any]) -> dict[str, Any]:
    """The printed line: ``full`` minus the per-cell lists, with the nested
    results folded to their headline figures."""
    line = {k: v for k, v in full.items()
            if k not in ("per_kernel", "extras", "selection", "decoder", "gpu_state")}
    line["selection"] = selection_summary(full.get("selection"))
    line["decoder"] = decoder_summary(full.get("decoder"))
    in_model = full.get("decode_in_model")
    if line["decoder"] is not None and in_model:
        line["decoder"]["library_in_model_us_per_step"] = in_model["step_library_us"]
    rows = list(full.get("per_kernel") or []) + list(full.get("extras") or [])
    line["prefill_floor"] = prefill_floor(rows) or None
    state = full.get("gpu_state") or {}
    pre = state.get("preflight") or {}
    line["gpu_idle_before"] = (not pre.get("busy")) if pre else None
    return line


def _reject_constant(name: str) -> float:
    raise ValueError(f"non-finite JSON constant {name}")


def dumps_line(line: dict[str, Any]) -> str:
    """Serialise the line as strict JSON (no NaN/Infinity), checked to parse
    back and to fit ``LINE_LIMIT``."""
    text = json.dumps(_finite(line), separators=(",", ":"), allow_nan=False)
    json.loads(text, parse_constant=_reject_constant)
    if len(text.encode()) >= LINE_LIMIT:
        raise ValueError(f"bench line is {len(text.encode())} bytes, limit {LINE_LIMIT}")
    return text


def _finite(obj: Any) -> Any:
    """NaN and infinities become null (JSON has no spelling for them)."""
    if isinstance(obj, float) and not math.isfinite(obj):
        return None
    if isinstance(obj, dict):
        return {k: _finite(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return [_finite(v) for v in obj]
    return obj


def cells_report(full: dict[str, Any], device: dict[str, Any], gpu_name: str,
                 comparisons: list[dict[str, Any]] | None = None) -> dict[str, Any]:
    """Every timed cell as a ``results`` row (kernel_name, shape, dtype,
    device, then the cell's figures), the selection rows as ``comparisons``,
    and the decoder breakdown under ``decoder``."""
    results = []
    for source in ("per_kernel", "extras"):
        for row in full.get(source) or []:
            cell = parse_cell(row["name"])
            results.append({
                "kernel_name": f"{cell['op']}_hip",
                "shape": cell["shape"],
                "dtype": cell["dtype"],
                "device": gpu_name,
                "cell": row["name"],
                "source": "headline step" if source == "per_kernel" else "extra cell",
                **{k: v for k, v in row.items() if k != "name"},
            })
    return _finite({
        "operation": "bench",
        "gpu": gpu_name,
        "device": device,
        "created_at": datetime.now(timezone.utc).isoformat(),
        "results": results,
        "comparisons": comparisons or [],
        "decoder": full.get("decoder"),
        "selection_not_hip": (full.get("selection") or {}).get("not_hip", []),
        "gpu_state": full.get("gpu_state"),
        "launch_floor": full.get("launch_floor"),
    })
