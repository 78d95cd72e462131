"""rocprofv3 output parsing on synthetic files (no GPU, no profiler).

The counter arithmetic is what ``bench.py``'s ``roofline.traffic`` rests on:
per-dispatch ``FETCH_SIZE`` / ``WRITE_SIZE`` (KiB, summed over the counter's
instances) are matched to the launch manifest from the end of the run, then
scaled by the reading of the plain elementwise reference of known traffic.
"""

from __future__ import annotations

import csv
import json
from pathlib import Path

import pytest

from ako_amd.benchmark import rocprof

COUNTER_FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _counter_csv(path: Path, counter: str, values_kib: list[list[float]]) -> Path:
    """One row per counter instance; dispatch i has the instance values values_kib[i]."""
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=COUNTER_FIELDS)
        w.writeheader()
        w.writerow({"Dispatch_Id": 0, "Kernel_Name": "setup", "Counter_Name": counter, "Counter_Value": 7})
        for i, parts in enumerate(values_kib, start=1):
            for v in parts:
                w.writerow({"Dispatch_Id": i, "Kernel_Name": f"k{i}", "Counter_Name": counter, "Counter_Value": v})
                w.writerow({"Dispatch_Id": i, "Kernel_Name": f"k{i}", "Counter_Name": "OTHER", "Counter_Value": 1e9})
    return path


def test_traffic_is_scaled_by_the_reference_kernel(tmp_path) -> None:
    gib = 1 << 30
    manifest = {"dispatches": [
        {"cell": "cell_a", "alg_bytes": 3 * (1 << 20)},
        {"cell": "cell_a", "alg_bytes": 3 * (1 << 20)},
        {"cell": "reference_neg_fp16_1GiB", "alg_bytes": 2 * gib},
    ]}
    (tmp_path / "m.json").write_text(json.dumps(manifest))
    # FETCH reads half scale (as on MI355X), WRITE full scale; two instances per dispatch.
    fetch = _counter_csv(tmp_path / "f.csv", "FETCH_SIZE", [[512, 512], [512, 512], [gib / 2048 / 2] * 2])
    write = _counter_csv(tmp_path / "w.csv", "WRITE_SIZE", [[512, 512], [512, 512], [gib / 1024 / 2] * 2])
    out = rocprof.traffic(fetch, write, tmp_path / "m.json")
    assert out["fetch_factor"] == pytest.approx(2.0) and out["write_factor"] == pytest.approx(1.0)
    cell = out["kernels"]["cell_a"]
    assert cell["fetch_bytes"] == 2 * (1 << 20) and cell["write_bytes"] == 1 << 20
    assert cell["traffic_over_alg"] == pytest.approx(1.0)
    # The markdown's machine-readable lines are what bench.py reads back.
    md = tmp_path / "t.md"
    md.write_text(rocprof.to_markdown(out, "cmd"))
    assert rocprof.load_traffic_md(md) == {"cell_a": cell["hbm_bytes_per_launch"]}


def test_traffic_rejects_a_short_run(tmp_path) -> None:
    manifest = {"dispatches": [{"cell": "c", "alg_bytes": 1}] * 3}
    (tmp_path / "m.json").write_text(json.dumps(manifest))
    f = _counter_csv(tmp_path / "f.csv", "FETCH_SIZE", [[1.0]])
    with pytest.raises(ValueError, match="manifest"):
        rocprof.traffic(f, f, tmp_path / "m.json")


def test_kernel_stats_and_trace_tail(tmp_path) -> None:
    stats = tmp_path / "s.csv"
    stats.write_text('"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"\n'
                     '"kern",4,400,100.0,80.0,90,110,5.0\n')
    rows = rocprof.read_kernel_stats(stats)
    assert rows[0]["calls"] == 4 and rows[0]["avg_ns"] == 100.0
    assert "| `kern` | 4 | 0.10 |" in rocprof.stats_markdown(rows, "cmd", "t")

    trace = tmp_path / "t.csv"
    with open(trace, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerow({"Kernel_Name": "warmup", "Start_Timestamp": 0, "End_Timestamp": 5_000_000})
        t = 10_000_000
        for _ in range(4):  # four steps of 1 ms: gemv 600 us, norm 100 us
            w.writerow({"Kernel_Name": "gemv", "Start_Timestamp": t, "End_Timestamp": t + 600_000})
            w.writerow({"Kernel_Name": "norm", "Start_Timestamp": t + 700_000, "End_Timestamp": t + 800_000})
            t += 1_000_000
    rows = rocprof.read_kernel_trace(trace)
    out = rocprof.tail_breakdown(rows, 4, tail_ms=3.9)
    by = {k["name"]: k for k in out["kernels"]}
    assert "warmup" not in by
    assert by["gemv"]["us_per_step"] == pytest.approx(600.0) and by["norm"]["calls_per_step"] == 1.0
    assert out["busy_us_per_step"] == pytest.approx(700.0)
    assert "| `gemv` | 1.0 | 600.0 |" in rocprof.breakdown_markdown(out, "cmd", "t")
    # Marker windows: norm ends each step; the last 3 steps lie between its 4th-last and last launch.
    marked = rocprof.tail_breakdown(rows, 3, marker="norm")
    assert marked["span_us_per_step"] == pytest.approx(1000.0)
    assert {k["name"]: k["calls_per_step"] for k in marked["kernels"]} == {"gemv": 1.0, "norm": 1.0}
    with pytest.raises(ValueError, match="need"):
        rocprof.tail_breakdown(rows, 9, marker="norm")
    # Timeline: the marked window opens at a norm's end, so each gemv takes the
    # 200 us gap before it plus its 600 us, each norm the 100 us gap plus 100 us.
    tl = {k["name"]: k for k in marked["kernels"]}
    assert tl["gemv"]["timeline_us_per_step"] == pytest.approx(800.0)
    assert tl["norm"]["timeline_us_per_step"] == pytest.approx(200.0)
    assert tl["norm"]["start_gap_us"] == pytest.approx(100.0)
    assert sum(k["timeline_us_per_step"] for k in marked["kernels"]) == pytest.approx(marked["span_us_per_step"])


def test_tail_breakdown_timeline_with_overlapping_records() -> None:
    """A short kernel whose recorded start falls inside the long kernel before
    it: its duration counts the overlap, its timeline share does not, and the
    timeline still sums to the span."""
    rows, t = [("mark", 0, 1000)], 1000
    for _ in range(3):  # gemv 600 us; ako kernel recorded from 50 us before gemv ends, 250 us long
        rows += [("gemv", t + 100_000, t + 700_000), ("_ZN3ako4norm", t + 650_000, t + 900_000),
                 ("mark", t + 950_000, t + 1_000_000)]
        t += 1_000_000
    out = rocprof.tail_breakdown(rows, 3, marker="mark")
    by = {k["name"]: k for k in out["kernels"]}
    assert by["_ZN3ako4norm"]["us_per_step"] == pytest.approx(250.0)
    assert by["_ZN3ako4norm"]["timeline_us_per_step"] == pytest.approx(200.0)
    assert by["_ZN3ako4norm"]["start_gap_us"] == pytest.approx(-50.0)
    assert out["library_timeline_us_per_step"] == pytest.approx(200.0)
    assert out["library_us_per_step"] == pytest.approx(250.0) and out["library_calls_per_step"] == 1.0
    assert sum(k["timeline_us_per_step"] for k in out["kernels"]) == pytest.approx(out["span_us_per_step"])
    assert "200.0 us of the step's timeline" in rocprof.breakdown_markdown(out, "cmd", "t")


def test_launch_window_cuts_the_event_timed_launches(tmp_path) -> None:
    """``--window`` averages exactly launches FIRST..FIRST+COUNT-1 of one kernel,
    counted in start order over that kernel alone, and sets the bench line's
    event figure beside them."""
    trace = tmp_path / "t.csv"
    with open(trace, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        t = 0
        for i in range(10):  # norm launch i lasts (i + 1) us; another kernel in between
            w.writerow({"Kernel_Name": "ako::norm<bf16>", "Start_Timestamp": t, "End_Timestamp": t + 1000 * (i + 1)})
            w.writerow({"Kernel_Name": "ako::norm<fp16>", "Start_Timestamp": t + 20_000, "End_Timestamp": t + 90_000})
            t += 100_000
    rows = rocprof.read_kernel_trace(trace)
    win = rocprof.launch_window(rows, "norm<bf16>", 4, 3)  # launches 4, 5, 6: 5, 6, 7 us
    assert (win["mean_us"], win["median_us"], win["min_us"], win["max_us"]) == (6.0, 6.0, 5.0, 7.0)
    assert win["launches_in_trace"] == 10
    with pytest.raises(ValueError, match="matches 2 kernels"):
        rocprof.launch_window(rows, "norm", 0, 1)
    with pytest.raises(ValueError, match="holds 10"):
        rocprof.launch_window(rows, "norm<bf16>", 8, 3)

    stats = tmp_path / "s.csv"
    stats.write_text('"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"\n'
                     '"ako::norm<bf16>",10,55000,5500.0,50.0,1000,10000,5.0\n')
    bench = tmp_path / "b.json"
    bench.write_text("noise\n" + json.dumps({"roofline": {"mean_launch_us": 6.6}}) + "\n")
    md = tmp_path / "o.md"
    assert rocprof.main(["--stats", str(stats), "--trace", str(trace), "--window", "norm<bf16>:4:3",
                         "--bench-json", str(bench), "--md", str(md)]) == 0
    text = md.read_text()
    assert "Launches 4-6 (0-based, of 10)" in text and "mean 6.00 us" in text
    assert "mean 6.60 us (`roofline.mean_launch_us`), +10.0%" in text


def test_counters_by_cell_averages_each_cell(tmp_path) -> None:
    manifest = {"dispatches": [{"cell": "a", "alg_bytes": 1}, {"cell": "a", "alg_bytes": 1},
                               {"cell": "b", "alg_bytes": 1}]}
    (tmp_path / "m.json").write_text(json.dumps(manifest))
    path = tmp_path / "c.csv"
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=COUNTER_FIELDS)
        w.writeheader()
        w.writerow({"Dispatch_Id": 0, "Kernel_Name": "setup", "Counter_Name": "X", "Counter_Value": 99})
        for did, (x, y) in enumerate([(1, 10), (3, 30), (5, 50)], start=1):
            for part in (x / 2, x / 2):  # two instances per dispatch
                w.writerow({"Dispatch_Id": did, "Kernel_Name": "k", "Counter_Name": "X", "Counter_Value": part})
            w.writerow({"Dispatch_Id": did, "Kernel_Name": "k", "Counter_Name": "Y", "Counter_Value": y})
    cells = rocprof.counters_by_cell(path, tmp_path / "m.json")
    assert cells == {"a": {"X": 2.0, "Y": 20.0}, "b": {"X": 5.0, "Y": 50.0}}
    assert "| a | 2 | 20 |" in rocprof.counters_markdown(cells, "cmd", "t")


def test_durations_by_grid_separate_launch_shapes(tmp_path) -> None:
    """One kernel launched at two grid sizes is two groups; warm-up launches drop per group."""
    trace = tmp_path / "t.csv"
    fields = ["Kernel_Name", "Workgroup_Size_X", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"]
    with open(trace, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=fields)
        w.writeheader()
        t = 0
        for dur_ns in (50_000, 10_000, 10_000, 12_000):  # the first is a slow warm-up
            w.writerow({"Kernel_Name": "rope", "Workgroup_Size_X": 256, "Grid_Size_X": 4096,
                        "Start_Timestamp": t, "End_Timestamp": t + dur_ns})
            t += 100_000
        for dur_ns in (90_000, 30_000, 40_000):
            w.writerow({"Kernel_Name": "rope", "Workgroup_Size_X": 256, "Grid_Size_X": 16384,
                        "Start_Timestamp": t, "End_Timestamp": t + dur_ns})
            t += 100_000
    groups = rocprof.durations_by_grid(trace, skip=1)
    assert [(g["grid"], g["calls"]) for g in groups] == [(4096, 3), (16384, 2)]
    assert groups[0]["median_us"] == pytest.approx(10.0) and groups[0]["min_us"] == pytest.approx(10.0)
    assert groups[1]["mean_us"] == pytest.approx(35.0)
    md = rocprof.grid_markdown(groups, "cmd", "t")
    assert "| `rope` | 256 | 16384 | 2 | 35.00 | 35.00 | 30.00 |" in md
    out = tmp_path / "g.md"
    assert rocprof.main(["--trace", str(trace), "--by-grid", "--skip", "1", "--md", str(out),
                         "--json", str(tmp_path / "g.json")]) == 0
    assert json.loads((tmp_path / "g.json").read_text())["kind"] == "durations_by_grid"


def test_durations_by_grid_split_into_runs(tmp_path) -> None:
    """A dynamic-shape kernel that launches one grid for two row widths: runs
    separated by a start gap come apart, warm-up drops per run, and a lone
    correctness launch is dropped by ``min_calls``."""
    trace = tmp_path / "t.csv"
    fields = ["Kernel_Name", "Workgroup_Size_X", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"]
    launches = [(0, 500_000)]  # a lone gate call, then two benchmarked cells
    t = 20_000_000
    for dur_ns in (150_000, 100_000, 100_000, 110_000):  # narrow rows
        launches.append((t, dur_ns))
        t += 300_000
    t += 20_000_000
    for dur_ns in (300_000, 200_000, 220_000, 200_000):  # wide rows, same grid
        launches.append((t, dur_ns))
        t += 600_000
    with open(trace, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=fields)
        w.writeheader()
        for start, dur in launches:
            w.writerow({"Kernel_Name": "triton_red_fused_x", "Workgroup_Size_X": 512, "Grid_Size_X": 8192,
                        "Start_Timestamp": start, "End_Timestamp": start + dur})
        w.writerow({"Kernel_Name": "other", "Workgroup_Size_X": 64, "Grid_Size_X": 64,
                    "Start_Timestamp": 5, "End_Timestamp": 6})
    groups = rocprof.durations_by_grid(trace, skip=1, run_gap_ms=5.0, min_calls=2)
    mine = [g for g in groups if g["name"] == "triton_red_fused_x"]
    assert [(g["run"], g["calls"]) for g in mine] == [(2, 3), (3, 3)]
    assert mine[0]["median_us"] == pytest.approx(100.0) and mine[1]["median_us"] == pytest.approx(200.0)
    # Without run splitting the two widths would share one median.
    whole = [g for g in rocprof.durations_by_grid(trace, skip=1) if g["name"] == "triton_red_fused_x"]
    assert len(whole) == 1 and "run" not in whole[0]
    md = rocprof.grid_markdown(groups, "cmd", "t", name_filter="triton,ako")
    assert "| `triton_red_fused_x` | 512 | 8192 | 3 | 3 | 200.00 | 206.67 |" in md and "`other`" not in md
    out = tmp_path / "g.md"
    assert rocprof.main(["--trace", str(trace), "--by-grid", "--skip", "1", "--run-gap-ms", "5",
                         "--min-calls", "2", "--filter", "triton,ako", "--md", str(out)]) == 0
    assert "| run |" in out.read_text()
