"""BASELINE.json configs[0], the CPU plumbing case: fp32 RMSNorm on CPU
through the unfused reference, x[2,128,1024] ~ N(0,1) seed 0,
weight[1024] ~ N(1, 0.1), eps 1e-6, y = x * rsqrt(mean(x^2) + eps) * w;
selection with the gate, a ulp report per candidate, and a cache write."""

from __future__ import annotations

import json

import numpy as np

from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.selector import KernelSelector
from ako_amd.ops._registry import register_all
from ako_amd.dispatcher.registry import KernelRegistry
from oracle import ops as oracle
from tests._util import randn


def test_config1_plumbing(tmp_path) -> None:
    import torch

    x = randn((2, 128, 1024), torch.float32, 0)
    w = randn((1024,), torch.float32, 1, scale=0.1, shift=1.0)
    cache_path = tmp_path / "kernel_cache.json"
    sel = KernelSelector(registry=register_all(KernelRegistry()), cache=KernelCache(path=cache_path),
                         allow_cpu_tuning=True, warmup=2, repeats=5)
    result = sel.select_entry("rmsnorm", x, w)

    # The winner is a baseline (the HIP candidate cannot run on CPU tensors) and
    # its output passes the gate against the oracle.
    assert result.source == "benchmark"
    assert result.entry.backend in ("pytorch", "torch_native")
    y = result.entry.fn(x, w, 1e-6)
    rep = oracle.gate(oracle.rmsnorm(x.numpy(), w.numpy(), 1e-6), y.numpy(), "float32")
    assert rep["passed"] and rep["err_ulps"] <= 4.0
    # Every gated candidate carries a ulp report; a HIP candidate is rejected, not fatal.
    assert all(r["passed"] for r in result.ulp_reports)
    assert all("requires a GPU tensor" in r for r in result.rejected if r.startswith("rmsnorm_hip"))
    # The decision was persisted with the reference's record format.
    doc = json.loads(cache_path.read_text())
    (gpu_key,) = doc["entries"]
    record = doc["entries"][gpu_key]["rmsnorm"]["(2, 128, 1024)_float32_(1024,)"]
    assert record["kernel"] == result.entry.kernel_name
    assert np.isfinite(record["error_budget"]) and record["backend"] == result.entry.backend
