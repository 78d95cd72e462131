"""The printed bench line: strict JSON, under the size limit, with the
headline keys; the per-cell report in the reference's report layout."""

from __future__ import annotations

import copy
import json
from pathlib import Path

import pytest

from ako_amd.benchmark.benchline import (
    LINE_LIMIT,
    cells_report,
    compact_line,
    dumps_line,
    parse_cell,
    prefill_floor,
)

ROOT = Path(__file__).resolve().parent.parent
#: A full result dict as bench.py assembled it before the per-cell lists moved
#: to the report file (a fixture of bench.py's own output): 20.5 KB as one
#: line, too long for a reader that keeps only the tail.
FULL = json.loads((ROOT / "tests" / "golden" / "bench_result_full.json").read_text())
#: The line the latest bench.py run printed.
LATEST = ROOT / "reports" / "mi355x" / "bench_latest.json"


def _full() -> dict:
    full = copy.deepcopy(FULL)
    rate = {"value": 12.1, "spread": [7.2, 21.3], "passes": 40}
    full["cpu_baseline"] = {
        **rate, "unit": "GB/s", "cores": 16, "os_cpu_count": 16, "kind": "port",
        "sample": "rmsnorm_ref/rmsnorm_residual_ref on host tensors, 512 of 16384 rows; median of passes",
        "full_size_check": {"cell": "rmsnorm_fp16_16384x4096", **rate},
        "per_op": {"rope_qk": {**rate, "cells": "q+k full size"}, "swiglu": {**rate, "cells": "[4096,14336]"}},
        "gpu_speedup": 540.0,
        "oracle_numpy": {**rate, "cores": 1, "cells": "64 rows"},
    }
    full["decode_in_model"] = {
        "ops": {op: {"graph_in_model_us": 2.7, "graph_cold_us": 2.6, "per_step": n}
                for op, n in (("rmsnorm", 1), ("rmsnorm_residual", 8), ("rope_qk_cache", 4), ("swiglu", 4))},
        "step_library_us": 45.0, "step_library_cold_us": 44.0, "calls_per_step": 17}
    full["selection"]["max_err_ulps"] = {"rmsnorm": 0.5, "rmsnorm_residual": 0.5, "rope": 0.0,
                                         "rope_qk": 0.0, "swiglu": 0.06}
    full["selection"]["not_hip"] = [{"cell": f"c{i}", "selected": "rmsnorm_torch_native",
                                     "latencies_us": {"a": 1.0, "b": 2.0}} for i in range(20)]
    return full


def _strict(text: str) -> dict:
    def reject(name: str) -> float:
        raise ValueError(name)

    return json.loads(text, parse_constant=reject)


def test_line_is_strict_json_under_the_limit() -> None:
    full = _full()
    assert len(json.dumps(full)) > LINE_LIMIT  # the fixture is the oversized line
    text = dumps_line(compact_line(full))
    line = _strict(text)
    assert len(text.encode()) < LINE_LIMIT * 3 // 4, len(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config"):
        assert key in line
    assert line["roofline"]["frac"] == FULL["roofline"]["frac"]
    assert line["roofline"]["copy_same_bytes"]["kernel_over_copy"] > 0
    assert line["cpu_baseline"]["per_op"]["swiglu"]["value"] == 12.1
    assert line["cpu_baseline"]["spread"] == [7.2, 21.3]
    sel = line["selection"]
    assert sel["cells"] == 59 and sel["not_hip"] == 20 and sel["max_err_ulps"]["swiglu"] == 0.06
    assert "per_kernel" not in line and "extras" not in line
    dec = line["decoder"]
    assert all(not isinstance(v, (dict, list)) for v in dec.values())  # one level
    assert dec["ako_prefill_ms"] == FULL["decoder"]["ako"]["prefill_ms"]
    assert dec["library_in_model_us_per_step"] == 45.0
    assert line["decode_in_model"]["ops"]["swiglu"]["per_step"] == 4


def test_line_rejects_non_finite_and_oversize() -> None:
    line = compact_line(_full())
    line["value"] = float("nan")
    assert _strict(dumps_line(line))["value"] is None
    line["padding"] = "x" * LINE_LIMIT
    with pytest.raises(ValueError, match="limit"):
        dumps_line(line)


def test_prefill_floor_picks_the_lowest_prefill_cell() -> None:
    floor = prefill_floor(FULL["per_kernel"] + FULL["extras"])
    assert floor["rmsnorm"]["cells"] == 6 and floor["rmsnorm_residual"]["cells"] == 6
    assert floor["swiglu"]["cells"] == 2 and floor["rope_qk"]["cells"] == 2
    lows = [r for r in FULL["extras"] if r["name"] in ("rope_qk_fp16_4x2048", "rope_qk_bf16_4x2048")]
    assert floor["rope_qk"]["min_pct"] == min(r["pct_hbm_peak"] for r in lows)
    # The step's cells count by their back-to-back figure, not the per-launch events.
    step = [r for r in FULL["per_kernel"] if r["name"].startswith("rmsnorm_fp16") or r["name"].startswith("rmsnorm_bf16")]
    assert floor["rmsnorm"]["min_pct"] == min(r["back_to_back"]["pct_hbm_peak"] for r in step)
    # The per-launch floor needs a per-launch figure on every cell of an op:
    # the step's cells have one at the top level, these extras none.
    assert floor["rmsnorm"]["min_per_launch_pct"] == min(r["pct_hbm_peak"] for r in step)
    assert "min_per_launch_pct" not in floor["rope_qk"]
    rows = copy.deepcopy(FULL["extras"])
    for r, p in zip((r for r in rows if r["name"] in ("rope_qk_fp16_4x2048", "rope_qk_bf16_4x2048")), (75.5, 76.2)):
        r["per_launch"] = {"pct_hbm_peak": p}
    floor2 = prefill_floor(rows)
    assert floor2["rope_qk"]["min_per_launch_pct"] == 75.5
    assert floor2["rope_qk"]["per_launch_cell"] == "rope_qk_fp16_4x2048"
    # decode cells never count
    for v in floor.values():
        shape = parse_cell(v["cell"])["shape"]
        assert shape[0] in (4096, 16384) or shape[:2] == [4, 2048], v


def test_parse_cell_names() -> None:
    assert parse_cell("rmsnorm_residual_fp16_16384x8192") == {
        "op": "rmsnorm_residual", "dtype": "float16", "shape": [16384, 8192], "variant": None}
    assert parse_cell("rope_q_bf16_4x2048x32x128")["shape"] == [4, 2048, 32, 128]
    c = parse_cell("rope_qk_cache_fp16_1x1_q32_kv32_slot511of640")
    assert c["op"] == "rope_qk_cache" and c["shape"] == [1, 1] and c["variant"] == "q32_kv32_slot511of640"
    assert parse_cell("rmsnorm_shard_partial_bf16_16384x2048_residual")["op"] == "rmsnorm_shard_partial"


def test_cells_report_layout() -> None:
    full = _full()
    comps = [{"operation": "rmsnorm", "shape": [1, 4096], "baseline_ms": 0.01, "candidate_ms": 0.002}]
    rep = _strict(json.dumps(cells_report(full, {"name": "gpu"}, "gpu", comps), allow_nan=False))
    assert set(rep) >= {"operation", "gpu", "device", "created_at", "results", "comparisons"}
    assert len(rep["results"]) == len(FULL["per_kernel"]) + len(FULL["extras"])
    row = rep["results"][0]
    assert row["kernel_name"].endswith("_hip") and row["shape"] and row["dtype"] in ("float16", "bfloat16")
    assert rep["comparisons"] == comps
    assert rep["decoder"]["ako"]["prefill_ms"] == FULL["decoder"]["ako"]["prefill_ms"]


def test_latest_recorded_line_is_within_the_contract() -> None:
    """The committed line of the latest bench.py run: strict JSON under the
    limit, with the headline keys, the roofline and the CPU baseline."""
    text = LATEST.read_text().strip()
    assert len(text) < LINE_LIMIT
    line = _strict(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and 0 < roof["frac"] < 1
    assert abs(roof["achieved"] / roof["peak"] - roof["frac"]) < 1e-3
    assert line["cpu_baseline"]["kind"] in ("port", "reference") and line["cpu_baseline"]["cores"] >= 1
