"""The persistent selection cache (``ako_amd.dispatcher.cache``).

What is pinned: the on-disk document is schema v2 exactly as the reference
writes it (``ako/dispatcher/cache.py:3-21``), so a cache file moves between the
two; records round-trip through disk; decisions are kept apart per GPU key
(the key now names the part, so two AMD parts never share decisions); v1
documents are upgraded; damage to the file never breaks dispatch.
"""

from __future__ import annotations

import json

from hypothesis import given, settings
from hypothesis import strategies as st

from ako_amd.dispatcher.cache import CACHE_SCHEMA_VERSION, KernelCache, default_cache_path

MI355X = "AMD_Radeon_Graphics_gfx950_256CU_2400MHz_288GB_0"
MI300X = "AMD_Radeon_Graphics_gfx942_304CU_2100MHz_192GB_0"
RMS_KEY = "(16384, 4096)_float16_(4096,)_float16"


def test_document_is_schema_v2(tmp_path) -> None:
    path = tmp_path / "kernel_cache.json"
    cache = KernelCache(path=path)
    cache.set(MI355X, "rmsnorm", RMS_KEY, "rmsnorm_hip", latency_p50_ms=0.05, baseline_ms=0.4,
              speedup=8.0, max_error=0.0, error_budget=5e-3, backend="hip")
    doc = json.loads(path.read_text())
    assert doc["version"] == CACHE_SCHEMA_VERSION == 2 and list(doc) == ["version", "entries"]
    record = doc["entries"][MI355X]["rmsnorm"][RMS_KEY]
    assert record["kernel"] == "rmsnorm_hip" and record["backend"] == "hip"
    assert record["speedup"] == 8.0 and isinstance(record["created_at"], str)
    assert cache.to_dict() == doc


def test_decisions_are_kept_per_gpu(tmp_path) -> None:
    cache = KernelCache(path=tmp_path / "c.json")
    cache.set(MI300X, "rmsnorm", RMS_KEY, "rmsnorm_torch_native")
    assert cache.get(MI355X, "rmsnorm", RMS_KEY) is None  # another part's decision is not reused
    cache.set(MI355X, "rmsnorm", RMS_KEY, "rmsnorm_hip")
    reloaded = KernelCache(path=tmp_path / "c.json")
    assert reloaded.get(MI300X, "rmsnorm", RMS_KEY) == "rmsnorm_torch_native"
    assert reloaded.get(MI355X, "rmsnorm", RMS_KEY) == "rmsnorm_hip"
    assert len(reloaded) == 2


_names = st.text("abcdefgh_0123456789()", min_size=1, max_size=12)


@settings(max_examples=40, deadline=None)
@given(st.lists(st.tuples(_names, _names, _names, _names,
                          st.one_of(st.none(), st.floats(0.0, 1e3, allow_nan=False))), max_size=12))
def test_records_round_trip_through_disk(tmp_path_factory, writes) -> None:
    path = tmp_path_factory.mktemp("rt") / "c.json"
    cache = KernelCache(path=path)
    expected = {}
    for gpu, op, shape, kernel, ms in writes:
        cache.set(gpu, op, shape, kernel, latency_p50_ms=ms)
        expected[(gpu, op, shape)] = (kernel, ms)
    reloaded = KernelCache(path=path)
    assert len(reloaded) == len(expected)
    for (gpu, op, shape), (kernel, ms) in expected.items():
        record = reloaded.get_record(gpu, op, shape)
        assert record["kernel"] == kernel
        assert ("latency_p50_ms" in record) == (ms is not None)  # None metrics are not stored
        if ms is not None:
            assert record["latency_p50_ms"] == ms


def test_v1_documents_are_upgraded(tmp_path) -> None:
    path = tmp_path / "c.json"
    path.write_text(json.dumps({MI300X: {"rmsnorm": {RMS_KEY: "rmsnorm_triton"},
                                         "rope": {"k": "rope_ref"}}}))
    cache = KernelCache(path=path)
    assert cache.get_record(MI300X, "rmsnorm", RMS_KEY) == {"kernel": "rmsnorm_triton"}
    assert len(cache) == 2
    cache.set(MI355X, "swiglu", "s", "swiglu_hip")
    doc = json.loads(path.read_text())
    assert doc["version"] == 2 and doc["entries"][MI300X]["rope"]["k"] == "rope_ref"
    assert KernelCache(path=path).get(MI300X, "rope", "k") == "rope_ref"


def test_damaged_files_never_break_lookups(tmp_path, caplog) -> None:
    path = tmp_path / "c.json"
    path.write_text('{"version": 2, "entries": {')
    cache = KernelCache(path=path)
    assert len(cache) == 0 and "Unreadable kernel cache" in caplog.text
    assert (tmp_path / "c.json.corrupt").read_text() == '{"version": 2, "entries": {'
    cache.set(MI355X, "rmsnorm", RMS_KEY, "rmsnorm_hip")
    assert KernelCache(path=path).get(MI355X, "rmsnorm", RMS_KEY) == "rmsnorm_hip"
    assert sorted(p.name for p in tmp_path.iterdir()) == ["c.json", "c.json.corrupt"]  # no temp files
    # Valid JSON of the wrong shape is ignored, not moved aside.
    path.write_text("[1, 2, 3]")
    assert len(KernelCache(path=path)) == 0 and path.read_text() == "[1, 2, 3]"
    path.write_text(json.dumps({"version": 2, "entries": ["x"]}))
    assert len(KernelCache(path=path)) == 0


def test_autosave_off_until_save(tmp_path) -> None:
    path = tmp_path / "sub" / "c.json"
    cache = KernelCache(path=path, autosave=False)
    cache.set(MI355X, "rmsnorm", RMS_KEY, "rmsnorm_hip")
    assert not path.exists()
    cache.save()
    assert KernelCache(path=path).get(MI355X, "rmsnorm", RMS_KEY) == "rmsnorm_hip"
    cache.clear()
    assert len(cache) == 0 and KernelCache(path=path).get(MI355X, "rmsnorm", RMS_KEY) == "rmsnorm_hip"


def test_hit_rate_and_location(tmp_path, monkeypatch) -> None:
    cache = KernelCache(path=tmp_path / "c.json")
    cache.set(MI355X, "rope", "a", "rope_hip")
    for key in ("a", "a", "b", "c"):
        cache.get(MI355X, "rope", key)
    stats = cache.stats()
    assert (stats.hits, stats.misses, stats.total) == (2, 2, 4)
    assert stats.to_dict() == {"hits": 2, "misses": 2, "lookups": 4, "hit_rate": 0.5}
    cache.clear()
    assert cache.stats().total == 0
    monkeypatch.setenv("AKO_CACHE_PATH", "~/ako-test/k.json")
    assert str(default_cache_path()).endswith("ako-test/k.json") and "~" not in str(default_cache_path())
    monkeypatch.delenv("AKO_CACHE_PATH")
    assert default_cache_path().parts[-2:] == (".ako", "kernel_cache.json")
