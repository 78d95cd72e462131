"""Registry and selector behaviour with plain Python candidates
(reference tests/test_dispatcher.py:39-213)."""

from __future__ import annotations

import json
import time
from pathlib import Path

import pytest
import torch

from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.hardware import get_device_info
from ako_amd.dispatcher.registry import KernelEntry, KernelRegistry
from ako_amd.dispatcher.selector import BASELINE_BACKENDS, KernelSelector, shape_key
from ako_amd.ops._registry import register_all
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref

REF = json.loads((Path(__file__).resolve().parent / "golden" / "reference_golden.json").read_text())


def _selector(tmp_path, registry, **kw) -> KernelSelector:
    return KernelSelector(registry=registry, cache=KernelCache(path=tmp_path / "cache.json"),
                          warmup=1, repeats=3, **kw)


def _registry(*entries) -> KernelRegistry:
    reg = KernelRegistry()
    for e in entries:
        reg.register(e)
    return reg


def _baseline(fn=rmsnorm_ref, priority=10) -> KernelEntry:
    return KernelEntry("rmsnorm", "rmsnorm_ref", fn, backend="pytorch", priority=priority)


def test_registry_basics() -> None:
    reg = _registry(_baseline(), _baseline())
    assert len(reg.list_kernels("rmsnorm")) == 1
    assert reg.list_ops() == ["rmsnorm"]
    assert reg.get("rmsnorm", "rmsnorm_ref") is not None
    assert reg.get("rmsnorm", "nope") is None and reg.default("nope") is None
    reg.register(KernelEntry("rmsnorm", "low", rmsnorm_ref, backend="hip", priority=1))
    assert reg.default("rmsnorm").kernel_name == "rmsnorm_ref"
    assert reg.unregister("rmsnorm", "low") and not reg.unregister("rmsnorm", "low")


def test_shape_key_format_matches_reference_records() -> None:
    """Keys of reports/rtx3070/selected_config_{fp16,bf16}.json of the reference."""
    for tag, dtype in (("fp16", torch.float16), ("bf16", torch.bfloat16)):
        rec = REF["selected_config_shape_keys"][tag]
        p = rec["parameters"]
        b, s, h = p["batch_size"], p["seq_len"], p["hidden_dim"]
        x = torch.empty(b, s, h, dtype=dtype)
        w = torch.empty(h, dtype=dtype)
        assert shape_key((x, w)) == rec["shape_keys"]["rmsnorm"]
        assert shape_key((x, x, w)) == rec["shape_keys"]["rmsnorm_residual"]
        q = torch.empty(b, s, p["num_heads"], p["head_dim"], dtype=dtype)
        t = torch.empty(s, p["head_dim"] // 2)
        assert shape_key((q, t, t), p["rope_style"]) == rec["shape_keys"]["rope"]
    x = torch.randn(2, 4)
    assert shape_key((x,)) != shape_key((x.half(),))
    with pytest.raises(ValueError):
        shape_key(())


def test_selector_default_and_unknown_op(tmp_path) -> None:
    sel = _selector(tmp_path, _registry(_baseline()), auto_tune=False)
    x, w = torch.randn(2, 16, 32), torch.ones(32)
    assert sel.select("rmsnorm", x, w)(x, w).shape == x.shape
    with pytest.raises(ValueError, match="No kernels registered"):
        _selector(tmp_path, KernelRegistry()).select("nope", torch.randn(2))


def test_selector_prefers_faster_valid_kernel(tmp_path) -> None:
    def slow(x, weight, eps=1e-6):
        time.sleep(0.002)
        return rmsnorm_ref(x, weight, eps)

    reg = _registry(_baseline(fn=slow), KernelEntry("rmsnorm", "fast", rmsnorm_ref, backend="hip", priority=5))
    result = _selector(tmp_path, reg, allow_cpu_tuning=True).select_entry("rmsnorm", torch.randn(2, 8, 32), torch.ones(32))
    assert result.entry.kernel_name == "fast"
    assert result.candidates_evaluated == 2 and result.speedup > 1.0


def test_selector_min_speedup_keeps_reference(tmp_path) -> None:
    reg = _registry(_baseline(), KernelEntry("rmsnorm", "same", rmsnorm_ref, backend="hip", priority=5))
    sel = _selector(tmp_path, reg, allow_cpu_tuning=True, min_speedup=1e6)
    assert sel.select_entry("rmsnorm", torch.randn(2, 8, 32), torch.ones(32)).entry.kernel_name == "rmsnorm_ref"


def test_selector_rejects_wrong_and_survives_broken(tmp_path) -> None:
    def wrong(x, weight, eps=1e-6):
        return torch.zeros_like(x)

    def broken(x, weight, eps=1e-6):
        raise RuntimeError("kernel launch failed")

    reg = _registry(_baseline(), KernelEntry("rmsnorm", "wrong", wrong, backend="hip", priority=5),
                    KernelEntry("rmsnorm", "broken", broken, backend="hip", priority=4))
    result = _selector(tmp_path, reg, allow_cpu_tuning=True).select_entry("rmsnorm", torch.randn(2, 8, 32), torch.ones(32))
    assert result.entry.kernel_name == "rmsnorm_ref"
    assert any(r.startswith("wrong: max_error=") for r in result.rejected)
    assert "broken: RuntimeError: kernel launch failed" in result.rejected


def test_selection_is_cached_with_reference_record_keys(tmp_path) -> None:
    reg = _registry(_baseline(), KernelEntry("rmsnorm", "alt", rmsnorm_ref, backend="hip", priority=5))
    sel = _selector(tmp_path, reg, allow_cpu_tuning=True)
    x, w = torch.randn(2, 8, 32), torch.ones(32)
    first = sel.select_entry("rmsnorm", x, w)
    second = sel.select_entry("rmsnorm", x, w)
    assert first.source == "benchmark" and second.source == "cache" and second.from_cache
    assert second.entry.kernel_name == first.entry.kernel_name
    assert sel.cache.stats().hits == 1
    record = sel.cache.get_record(get_device_info(x.device).cache_key, "rmsnorm", shape_key((x, w)))
    assert set(record) == {"kernel", "created_at", "latency_p50_ms", "baseline_ms", "speedup",
                           "best_baseline_ms", "best_baseline_kernel", "speedup_vs_best_baseline",
                           "max_error", "error_budget", "backend"}


def test_memo_hot_path(tmp_path) -> None:
    sel = _selector(tmp_path, _registry(_baseline()), auto_tune=False)
    w = torch.ones(32)
    x = torch.randn(2, 8, 32)
    for _ in range(5):
        sel.select("rmsnorm", x, w)
    assert sel.cache.stats().total == 1
    sel.clear_memo()
    sel.select("rmsnorm", x, w)
    sel.select("rmsnorm", torch.randn(4, 8, 32), w)
    sel.select("rmsnorm", x.half(), w)
    sel.select("rmsnorm", x, w, extra_key="variant")
    assert sel.cache.stats().total == 5


def test_forced_kernel_bypasses_cache(tmp_path) -> None:
    reg = _registry(_baseline(), KernelEntry("rmsnorm", "alt", rmsnorm_ref, backend="hip", priority=5))
    sel = _selector(tmp_path, reg, allow_cpu_tuning=True)
    result = sel.select_entry("rmsnorm", torch.randn(2, 8, 32), torch.ones(32), forced="alt")
    assert (result.entry.kernel_name, result.source, len(sel.cache)) == ("alt", "forced", 0)
    with pytest.raises(ValueError, match="Unknown kernel"):
        sel.select_entry("rmsnorm", torch.randn(2, 8, 32), torch.ones(32), forced="nope")


def test_selection_result_to_dict(tmp_path) -> None:
    payload = _selector(tmp_path, _registry(_baseline()), auto_tune=False).select_entry(
        "rmsnorm", torch.randn(2, 4), torch.ones(4)).to_dict()
    assert (payload["selected_kernel"], payload["operation"], payload["source"]) == ("rmsnorm_ref", "rmsnorm", "default")
    assert payload["ulp_reports"] == []


def test_register_all_covers_every_op_with_safe_defaults() -> None:
    reg = register_all(KernelRegistry())
    # The reference's four operations, plus the one-launch query/key pair.
    assert reg.list_ops() == ["rmsnorm", "rmsnorm_residual", "rope", "rope_qk", "swiglu"]
    for op in reg.list_ops():
        assert reg.default(op).backend == "pytorch"
        pytorch = [k for k in reg.list_kernels(op) if k.backend == "pytorch"]
        assert len(pytorch) == 1
    assert "torch_native" in BASELINE_BACKENDS and "hip" not in BASELINE_BACKENDS
    # No Triton backend anywhere.
    assert all(k.backend != "triton" for op in reg.list_ops() for k in reg.list_kernels(op))


def test_register_all_hip_candidates_and_opt_out(monkeypatch) -> None:
    from ako_amd import _native

    reg = register_all(KernelRegistry())
    if _native.is_available():
        for op in ("rmsnorm", "rmsnorm_residual", "rope", "rope_qk", "swiglu"):
            hip = [k for k in reg.list_kernels(op) if k.backend == "hip"]
            assert [k.kernel_name for k in hip] == [f"{op}_hip"] and hip[0].priority == 5
    monkeypatch.setenv("AKO_HIP_DISABLE", "1")
    reg = register_all(KernelRegistry())
    assert all(k.backend != "hip" for op in reg.list_ops() for k in reg.list_kernels(op))


def test_compile_baselines_are_opt_in(monkeypatch) -> None:
    monkeypatch.delenv("AKO_ENABLE_COMPILE", raising=False)
    reg = register_all(KernelRegistry())
    assert all(k.backend != "torch_compile" for op in reg.list_ops() for k in reg.list_kernels(op))
    monkeypatch.setenv("AKO_ENABLE_COMPILE", "1")
    reg = register_all(KernelRegistry())
    for op in ("rmsnorm", "rmsnorm_residual", "rope", "swiglu"):
        assert reg.get(op, f"{op}_compiled").backend == "torch_compile"


def test_device_info_cpu() -> None:
    info = get_device_info(torch.device("cpu"))
    assert (info.device_type, info.compute_backend, info.cache_key) == ("cpu", "cpu", "cpu_-1")


# HIP's answers for three parts that all report the generic marketing name:
# (gcnArchName, CUs, peak engine clock kHz, HBM bytes).
_PARTS = {
    "mi300x": ("gfx942:sramecc+:xnack-", 304, 2_100_000, 192 * 1024**3),
    "mi350x": ("gfx950:sramecc+:xnack-", 256, 2_200_000, 288 * 1024**3),
    "mi355x": ("gfx950:sramecc+:xnack-", 256, 2_400_000, 288 * 1024**3),
}


def _fake_rocm_device(monkeypatch, part: str, *, library: bool = True,
                      name: str = "AMD Radeon Graphics"):
    from functools import lru_cache
    from types import SimpleNamespace

    from ako_amd.dispatcher import hardware

    arch, cus, clock, mem = _PARTS[part]
    props = SimpleNamespace(name=name, major=9, minor=5, total_memory=mem,
                            multi_processor_count=cus, gcnArchName=arch, L2_cache_size=4 << 20,
                            regs_per_multiprocessor=524288, shared_memory_per_block=65536)
    ident = {"name": name, "arch": arch, "cus": str(cus), "clock_khz": str(clock),
             "mem_bytes": str(mem), "hip_driver": "70226015"}
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda i: props)
    monkeypatch.setattr(torch.version, "hip", "7.0.51831", raising=False)
    monkeypatch.setattr(hardware, "_hip_identity", lambda i: ident if library else None)
    monkeypatch.setattr(hardware, "_amdgpu_module_version", lru_cache(maxsize=1)(lambda: None))
    hardware.clear_device_cache()
    return hardware


def test_cache_key_tells_amd_parts_apart(monkeypatch) -> None:
    """The generic HIP name alone would give every part the same key; the ISA,
    CU count, clock and HBM size make each part's key its own."""
    keys = {}
    for part in _PARTS:
        hardware = _fake_rocm_device(monkeypatch, part)
        info = hardware.get_device_info("cuda:0")
        keys[part] = info.cache_key
        assert info.marketing_name == "AMD Radeon Graphics"
        assert info.driver_version == "hip 70226015"
    assert keys["mi355x"] == "AMD_Radeon_Graphics_gfx950_256CU_2400MHz_288GB_0"
    assert keys["mi300x"] == "AMD_Radeon_Graphics_gfx942_304CU_2100MHz_192GB_0"
    assert len(set(keys.values())) == 3
    # Without the library the clock comes from the card's pp_dpm_sclk, and
    # the key is the one the library gives.
    hardware = _fake_rocm_device(monkeypatch, "mi300x", library=False)
    monkeypatch.setattr(hardware, "sysfs_clock_khz", lambda i: 2_100_000)
    assert hardware.get_device_info("cuda:0").cache_key == keys["mi300x"]
    # With neither source: no clock, still the ISA, and the short key is not
    # memoised, so the full key appears as soon as a source does.
    hardware = _fake_rocm_device(monkeypatch, "mi300x", library=False)
    monkeypatch.setattr(hardware, "sysfs_clock_khz", lambda i: None)
    assert hardware.get_device_info("cuda:0").cache_key == "AMD_Radeon_Graphics_gfx942_304CU_192GB_0"
    monkeypatch.setattr(hardware, "sysfs_clock_khz", lambda i: 2_100_000)
    assert hardware.get_device_info("cuda:0").cache_key == keys["mi300x"]
    monkeypatch.setattr(hardware, "sysfs_clock_khz", lambda i: None)
    assert hardware.get_device_info("cuda:0").cache_key == keys["mi300x"]  # now memoised
    hardware.clear_device_cache()


def test_driver_label_prefers_the_module_version() -> None:
    from ako_amd.dispatcher.hardware import driver_label, part_label

    assert driver_label("6.10.5", 70226015) == "amdgpu 6.10.5"
    assert driver_label(None, 70226015) == "hip 70226015"
    assert driver_label(None, None) is None
    assert part_label("AMD Instinct MI355X", "gfx950:xnack-", 256, 2_400_000, None) == \
        "AMD Instinct MI355X gfx950 256CU 2400MHz"
    # An empty name and the generic one describe the same part: one label, one cache key.
    generic = {part_label(n, "gfx950:sramecc+:xnack-", 256, 2_400_000, 288 << 30)
               for n in ("", "  ", "AMD Radeon Graphics", "AMD GPU")}
    assert generic == {"AMD Radeon Graphics gfx950 256CU 2400MHz 288GB"}


def test_empty_hip_name_keeps_the_generic_cache_key(monkeypatch) -> None:
    """A box whose HIP runtime reports an empty device name finds the
    selections cached under the generic name for the same part."""
    hardware = _fake_rocm_device(monkeypatch, "mi355x")
    generic = hardware.get_device_info("cuda:0").cache_key
    for library in (True, False):
        hardware = _fake_rocm_device(monkeypatch, "mi355x", library=library, name="")
        monkeypatch.setattr(hardware, "sysfs_clock_khz", lambda i: 2_400_000)
        assert hardware.get_device_info("cuda:0").cache_key == generic
    hardware.clear_device_cache()


def test_reference_test_hooks(tmp_path, monkeypatch) -> None:
    """The reset/clear helpers the reference exposes for tests, and
    ``load_baseline`` for its regression diffs, behave as their names say."""
    from ako_amd.benchmark.profiler import kernel_table, profile_cuda
    from ako_amd.dispatcher import hardware
    from ako_amd.ops import _registry, rmsnorm_torch
    from ako_amd.validation.regression import load_baseline

    register_all()
    assert _registry._registered
    _registry.reset_registration()
    assert not _registry._registered
    register_all()
    assert _registry._registered

    rmsnorm_torch._compiled["probe"] = object()
    rmsnorm_torch.reset_compiled_cache()
    assert rmsnorm_torch._compiled == {}

    first = get_device_info("cpu")
    assert len(hardware._INFO_CACHE) >= 1
    hardware.clear_device_cache()
    assert len(hardware._INFO_CACHE) == 0
    assert get_device_info("cpu") == first

    path = tmp_path / "baseline.json"
    path.write_text(json.dumps({"comparisons": [{"shape": [1, 2], "selected_kernel": "k"}]}))
    assert load_baseline(path)["comparisons"][0]["selected_kernel"] == "k"

    with profile_cuda() as prof:
        torch.ones(4).sum()
    assert any("sum" in e.name for e in prof.events())
    rows = kernel_table(prof)  # host op time on a CPU-only run
    assert rows and any("sum" in r["name"] for r in rows)
    assert abs(sum(r["share"] for r in rows) - 1.0) < 1e-9


def test_kernel_table_counts_device_kernels_once() -> None:
    """A host op that launched kernels also reports their device time; the
    device table keeps the kernels only, so nothing counts twice."""
    from types import SimpleNamespace

    from torch.autograd import DeviceType

    from ako_amd.benchmark.profiler import kernel_table

    events = [SimpleNamespace(key="aten::mm", count=2, self_device_time_total=50.0, device_type=DeviceType.CPU),
              SimpleNamespace(key="Cijk_gemm", count=2, self_device_time_total=50.0, device_type=DeviceType.CUDA),
              SimpleNamespace(key="_ZN3ako11rmsnorm_reg", count=1, self_device_time_total=10.0,
                              device_type=DeviceType.CUDA)]
    prof = SimpleNamespace(key_averages=lambda: events)
    rows = kernel_table(prof, device=True)
    assert [r["name"] for r in rows] == ["Cijk_gemm", "_ZN3ako11rmsnorm_reg"]
    assert sum(r["total_us"] for r in rows) == 60.0


def test_library_share_counts_ako_kernels() -> None:
    from ako_amd.benchmark.profiler import library_share, table_markdown

    rows = [{"name": "void ako::rmsnorm_reg<_Float16, 4, 2>(ako::RmsDev)", "calls": 9, "total_us": 30.0, "share": 0.3},
            {"name": "Cijk_Alik_Bljk_HHS_BH", "calls": 29, "total_us": 60.0, "share": 0.6},
            {"name": "_ZN3ako11swiglu_flatIDF16_Li1ELi256EEEvPKT_S3_PS1_lll", "calls": 4, "total_us": 10.0,
             "share": 0.1}]
    share = library_share(rows)
    assert share["share"] == 0.4 and share["library_calls"] == 13 and len(share["library_kernels"]) == 2
    md = table_markdown(rows, per=1)
    assert md.count("\n") == 4 and "30.0" in md
