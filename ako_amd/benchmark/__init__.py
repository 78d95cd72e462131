"""Measurement: per-op timing, graphs, reports, HBM roofline, rocprofv3 counters."""

from ako_amd.benchmark.bench_op import bench_op, bench_shapes, parse_dtypes
from ako_amd.benchmark.report import BenchmarkReport, save_report

__all__ = ["BenchmarkReport", "bench_op", "bench_shapes", "parse_dtypes", "save_report"]
