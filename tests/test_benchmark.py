"""Measurement utilities on the CPU: bench_op semantics, statistics, reports,
graph capture fallbacks, regression diffs, roofline arithmetic."""

from __future__ import annotations

import json
import random
import statistics
import time

import pytest
import torch

from ako_amd.benchmark import roofline as rf
from ako_amd.benchmark.bench_op import (
    MAX_INNER_ITERS,
    MAX_RING_COPIES,
    UNSTABLE_CV,
    BenchResult,
    InputRing,
    bench_op,
    bootstrap_ci,
    bootstrap_ratio_ci,
    compare_paired,
    parse_dtypes,
    percentile,
    ring_state,
)
from ako_amd.benchmark.env import host_cpu, sample_env
from ako_amd.benchmark.graph import capture_calls
from ako_amd.benchmark.report import BenchmarkReport
from ako_amd.dispatcher.hardware import get_device_info
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref
from ako_amd.ops.rope_ref import build_rope_tables, rope_ref
from ako_amd.validation.regression import compare_bench_lines, compare_reports
from ako_amd.validation import regression


def test_bench_op_cpu_basics() -> None:
    x, w = torch.randn(4, 64, 128), torch.ones(128)
    r = bench_op(rmsnorm_ref, (x, w), warmup=2, repeats=5, kernel_name="ref")
    assert r.latency_p50_ms > 0 and r.kernel_name == "ref" and len(r.samples_ms) == 5
    assert r.latency_p95_ms >= r.latency_p50_ms
    assert r.gpu_p50_ms is None and r.launch_overhead_ms is None and r.l2_state == "n/a"
    assert "gpu_p50_ms" not in r.to_dict()


def test_bench_op_call_kwargs_and_inner() -> None:
    x = torch.randn(1, 8, 2, 16)
    cos, sin = build_rope_tables(8, 16)
    r = bench_op(rope_ref, (x, cos, sin), warmup=1, repeats=3, call_kwargs={"style": "interleaved"}, inner=3)
    assert r.dtype == "float32" and r.inner_iters == 3
    small = bench_op(rmsnorm_ref, (torch.randn(8, 8), torch.ones(8)), warmup=2, repeats=3)
    assert 1 < small.inner_iters <= MAX_INNER_ITERS


def test_bench_op_runs() -> None:
    x, w = torch.randn(2, 16, 32), torch.ones(32)
    single = bench_op(rmsnorm_ref, (x, w), warmup=1, repeats=4)
    assert len(single.run_p50s) == 1 and single.to_dict()["runs"] == 1
    many = bench_op(rmsnorm_ref, (x, w), warmup=1, repeats=4, runs=3)
    assert len(many.run_p50s) == 3 and len(many.samples_ms) == 12 and many.iqr_ms >= 0


def test_launch_overhead_not_clamped() -> None:
    r = BenchResult("k", (1,), "float16", "cuda:0", 1.0, 1.0, 1.0, 0.0, [1.0], gpu_p50_ms=1.25)
    assert r.launch_overhead_ms == pytest.approx(-0.25)
    assert r.to_dict()["launch_overhead_ms"] == pytest.approx(-0.25)


def test_cv_flag() -> None:
    noisy = BenchResult("k", (1,), "f", "cpu", 1, 1, 1, 1, [1.0], run_p50s=(1.0, 2.0, 3.0, 0.5, 4.0))
    assert noisy.cv > UNSTABLE_CV and noisy.to_dict()["unstable"] is True
    calm = BenchResult("k", (1,), "f", "cpu", 1, 1, 1, 1, [1.0], run_p50s=(1.0, 1.02, 0.99, 1.01, 0.98))
    assert not calm.unstable and calm.iqr_ms == pytest.approx(0.02)


def test_bootstrap_intervals() -> None:
    rng = random.Random(1234)
    ratios = [1.4 * (1 + rng.uniform(-0.1, 0.1)) / (1 + rng.uniform(-0.1, 0.1)) for _ in range(30)]
    low, high = bootstrap_ci(ratios, seed=0)
    assert 1.0 < low < 1.4 < high
    assert bootstrap_ci([]) == (0.0, 0.0)
    slow = [1.4 * (1 + rng.uniform(-0.1, 0.1)) for _ in range(40)]
    fast = [1 + rng.uniform(-0.1, 0.1) for _ in range(40)]
    ratio, lo, hi = bootstrap_ratio_ci(slow, fast)
    assert 1.0 < lo <= ratio <= hi
    with pytest.raises(ValueError):
        bootstrap_ratio_ci([], fast)


def test_compare_paired_on_cpu() -> None:
    x, w = torch.randn(2, 16, 32), torch.ones(32)
    out = compare_paired(rmsnorm_ref, rmsnorm_ref, (x, w), pairs=3, warmup=1, repeats=3)
    low, high = out["speedup_ci95"]
    assert out["pairs"] == 3 and low <= out["speedup_median"] <= high


def test_parse_dtypes() -> None:
    assert parse_dtypes(["fp16", "bf16", "fp32"]) == [torch.float16, torch.bfloat16, torch.float32]
    with pytest.raises(ValueError, match="Unknown dtype"):
        parse_dtypes(["int8"])


def test_report_and_regression_diff() -> None:
    report = BenchmarkReport(operation="rmsnorm", device=get_device_info("cpu"))
    report.add_comparison(shape=[8, 2048, 4096], baseline_ms=1.2, candidate_ms=0.3, max_error=1e-4,
                          selected_kernel="rmsnorm_hip", dtype="float16", best_baseline_ms=0.45,
                          best_baseline_kernel="rmsnorm_torch_native", gbps=123.0)
    row = report.to_dict()["comparisons"][0]
    assert row["speedup"] == 4.0 and row["speedup_vs_best_baseline"] == 1.5 and row["gbps"] == 123.0
    slower = {"comparisons": [dict(row, candidate_ms=0.4)]}
    assert compare_reports(slower, report.to_dict())
    other_dtype = {"comparisons": [dict(row, candidate_ms=0.4, dtype="bfloat16")]}
    assert compare_reports(other_dtype, report.to_dict()) == []


def test_report_carries_counters_without_changing_its_layout() -> None:
    report = BenchmarkReport(operation="rmsnorm", device=get_device_info("cpu"))
    report.add_comparison(shape=[16384, 4096], baseline_ms=1.0, candidate_ms=0.05, max_error=0.0,
                          selected_kernel="rmsnorm_hip", cell="rmsnorm_fp16_16384x4096")
    plain = report.to_dict()
    assert "counters" not in plain  # the reference's keys only, until counters are attached
    traffic = {"reference": "reference_neg_fp16_1GiB", "fetch_factor": 2.0, "write_factor": 1.0,
               "kernels": {"rmsnorm_fp16_16384x4096": {"alg_bytes": 268443648, "fetch_bytes": 134322434,
                                                       "write_bytes": 134218794, "hbm_bytes_per_launch": 268541228,
                                                       "traffic_over_alg": 1.0004}}}
    report.attach_counters(traffic)
    out = report.to_dict()
    assert out["counters"]["fetch_factor"] == 2.0
    assert out["comparisons"][0]["traffic_over_alg"] == 1.0004
    assert set(plain) <= set(out)


def _bench_line(value=6300.0, gbps=6000.0, graph_us=2.0, decode=0.78) -> dict:
    return {"metric": "m", "value": value, "higher_is_better": True,
            "per_kernel": [{"name": "rmsnorm_fp16_16384x4096", "gbps": gbps}],
            "extras": [{"name": "rmsnorm_fp16_1x4096", "gbps": 3.6, "graph_us": graph_us}],
            "decoder": {"ako": {"prefill_ms": 1.7, "decode_ms_per_step": 1.1,
                                "graphed_decode_ms_per_step": decode}}}


def test_bench_line_regression_diff(tmp_path) -> None:
    base = _bench_line()
    assert compare_bench_lines(_bench_line(), base) == []
    assert compare_bench_lines(_bench_line(value=6350.0, gbps=6100.0, graph_us=1.9, decode=0.7), base) == []
    warnings = compare_bench_lines(_bench_line(value=5000.0, gbps=5000.0, graph_us=3.0, decode=0.9), base)
    assert len(warnings) == 4
    assert any("graph_us" in w for w in warnings) and any("graphed_decode" in w for w in warnings)
    assert compare_bench_lines({**_bench_line(), "metric": "other"}, base)[0].startswith("Different")
    # The command line reads the last JSON line of each file and fails on a regression.
    cur, old = tmp_path / "cur.json", tmp_path / "old.json"
    old.write_text("[bench] log line\n" + json.dumps(base) + "\n")
    cur.write_text(json.dumps(_bench_line(value=5000.0)) + "\n")
    assert regression.main([str(cur), str(old)]) == 1
    assert regression.main([str(old), str(old)]) == 0
    pretty = tmp_path / "pretty.json"  # an indented record, as committed under reports/
    pretty.write_text(json.dumps(base, indent=1))
    assert regression.main([str(old), str(pretty)]) == 0


def test_graph_capture_is_a_noop_on_cpu() -> None:
    cap = capture_calls(lambda t: t @ t, [(torch.randn(8, 8),)])
    assert cap.graph is None and cap.calls == 0 and "not on a GPU" in cap.reason
    with pytest.raises(RuntimeError, match="nothing was captured"):
        cap.replay()
    assert capture_calls(lambda t: t, []).reason == "no calls to capture"
    r = bench_op(lambda t: t @ t, (torch.randn(16, 16),), warmup=1, repeats=2, graph=True)
    assert r.graph_captured == 0


def test_input_ring_rotates_copies_of_contiguous_tensors() -> None:
    x, w = torch.randn(3, 5), torch.randn(5)
    strided = torch.randn(4, 10)[:, ::2]
    ring = InputRing((x, w, strided, 7), 4)
    assert len(ring) == 4 and ring.shared == 1
    seen = [ring.next() for _ in range(5)]
    assert seen[0][0] is x and seen[4][0] is x  # entry 0 is the caller's, then it wraps
    for entry in seen[1:4]:
        assert torch.equal(entry[0], x) and entry[0].data_ptr() != x.data_ptr()
        assert torch.equal(entry[1], w) and entry[1].data_ptr() != w.data_ptr()
        assert entry[2] is strided and entry[3] == 7  # strided and non-tensors are shared
    assert len({e[0].data_ptr() for e in seen[:4]}) == 4
    assert InputRing((x,), 1).entries == [(x,)]


def test_ring_state_and_percentile() -> None:
    l2, mall = 32 << 20, 256 << 20
    assert ring_state(2 * (l2 + mall), l2, mall) == "cold"
    assert ring_state(2 * l2, l2, mall) == "l2-cold"
    assert ring_state(l2, l2, mall) == "warm"
    assert MAX_RING_COPIES >= 256
    assert percentile([], 0.5) == 0.0
    assert percentile([3.0, 1.0, 2.0], 0.5) == 2.0
    assert percentile([1.0, 2.0, 3.0, 4.0], 0.5) == 2.0  # nearest rank: lower median
    assert percentile([1.0, 2.0, 3.0, 4.0], 0.95) == 4.0 and percentile([5.0], 0.0) == 5.0


def test_compare_paired_sees_a_real_difference() -> None:
    # Sleeps rather than compute: a sleep only ever overshoots, so the 8:1
    # ratio cannot collapse under load from other processes on the host (a
    # compute-bound pair with a 4:1 ratio once measured under 2x there).
    x, w = torch.randn(4, 8), torch.ones(8)

    def slow(a, b):
        time.sleep(0.008)

    def fast(a, b):
        time.sleep(0.001)

    out = compare_paired(slow, fast, (x, w), pairs=5, warmup=1, repeats=4)
    assert out["speedup_median"] > 2.0 and out["significant"]
    assert out["speedup_ci95"][0] <= out["speedup_median"] <= out["speedup_ci95"][1]


def test_roofline_bytes_and_peaks() -> None:
    assert rf.alg_bytes_rmsnorm(16384, 4096, torch.float16) == 2 * 16384 * 4096 * 2 + 4096 * 2
    assert rf.alg_bytes_rmsnorm_residual(2, 8, torch.bfloat16, torch.float32) == 4 * 2 * 8 * 2 + 8 * 4
    assert rf.alg_bytes_rope(4, 2048, 32, 128, torch.bfloat16, torch.float32) == 2 * 4 * 2048 * 32 * 128 * 2 + 2 * 2048 * 64 * 4
    assert rf.alg_bytes_swiglu(16384, 14336, torch.bfloat16) == 3 * 16384 * 14336 * 2
    assert rf.HBM_PEAK_GBPS["gfx950"] == 8000.0
    assert rf.copies_for_cold(1) > 100 and rf.copies_for_cold(10**10) == 2
    stats = rf.LaunchStats("k", 8_000_000_000, [1.0, 1.0])
    assert stats.gbps() == pytest.approx(8000.0) and stats.to_dict(8000.0)["pct_hbm_peak"] == 100.0


def test_env_samples_degrade_to_none() -> None:
    sample = sample_env(index=99)
    assert set(sample) == {"sm_clock_mhz", "temp_c", "power_w", "throttle_reasons"}
    assert all(v is None for v in sample.values())
    assert host_cpu()["os_cpu_count"] >= 1


def test_copy_ceiling_lines_pick_the_fastest_shape(monkeypatch, tmp_path) -> None:
    text = ("noise\n"
            '{"bytes_per_buffer": 64, "traffic_bytes": 128, "block": 256, "us": 2.0, "gbps": 0.064, "frac": 0.1, '
            '"b2b_us": 1.0, "b2b_gbps": 0.128, "b2b_frac": 0.3}\n'
            '{"bytes_per_buffer": 64, "traffic_bytes": 128, "block": 1024, "us": 1.0, "gbps": 0.128, "frac": 0.2, '
            '"b2b_us": 1.5, "b2b_gbps": 0.085, "b2b_frac": 0.25}\n')
    best = rf.parse_copy_ceiling(text)
    assert best["block"] == 1024 and best["frac"] == 0.2
    # The fastest back-to-back copy may be another shape: reported beside it.
    assert best["best_b2b_frac"] == 0.3 and best["best_b2b_gbps"] == 0.128
    assert rf.parse_copy_ceiling("no json here") is None
    # Without the built probe the figure is simply absent.
    import ako_amd._build as build

    monkeypatch.setattr(build, "COPY_PROBE_PATH", tmp_path / "missing")
    assert rf.copy_same_bytes(1 << 20) is None


def test_bench_refuses_more_than_one_gpu() -> None:
    """bench.py measures one GPU; asked for more it exits 2 and says why."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    out = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "4"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 2
    assert "measures one GPU" in out.stderr and out.stdout == ""


def test_ring_plan_covers_the_caches_within_free_memory(monkeypatch) -> None:
    """On a GPU the ring wants 2 x (L2 + MALL) bytes of copies; it is capped
    at MAX_RING_COPIES and at a quarter of the free device memory, and its
    l2_state says what it reaches (device queries faked, no GPU needed)."""
    import importlib

    bo = importlib.import_module("ako_amd.benchmark.bench_op")  # the module, not the function
    l2, mall = 32 << 20, 256 << 20
    monkeypatch.setattr(bo, "cache_bytes", lambda device: (l2, mall))
    gpu = torch.device("cuda", 0)
    x = torch.empty(4 << 20, dtype=torch.int8)  # 4 MiB per call
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (64 << 30, 288 << 30))
    assert bo.plan_ring((x,), gpu, cold=True) == (144, "cold")  # 576 MiB / 4 MiB
    assert bo.plan_ring((x,), gpu, cold=False) == (1, "warm")
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (512 << 20, 288 << 30))
    assert bo.plan_ring((x,), gpu, cold=True) == (32, "l2-cold")  # 128 MiB: a quarter of 512 MiB
    tiny = torch.empty(64, dtype=torch.int8)
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (64 << 30, 288 << 30))
    assert bo.plan_ring((tiny,), gpu, cold=True) == (bo.MAX_RING_COPIES, "warm")
    assert bo.plan_ring((x,), torch.device("cpu"), cold=True) == (1, "n/a")
