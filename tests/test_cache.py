"""The persistent decision cache (reference tests/test_cache.py:10-79)."""

from __future__ import annotations

import json

from ako_amd.dispatcher.cache import CACHE_SCHEMA_VERSION, KernelCache, default_cache_path


def test_records_carry_metrics(tmp_path) -> None:
    cache = KernelCache(path=tmp_path / "cache.json")
    cache.set("MI355X_0", "rmsnorm", "fp16_8x2048", "rmsnorm_hip", speedup=1.56, max_error=3e-4, skipped=None)
    record = cache.get_record("MI355X_0", "rmsnorm", "fp16_8x2048")
    assert record["kernel"] == "rmsnorm_hip"
    assert record["speedup"] == 1.56
    assert "created_at" in record and "skipped" not in record


def test_persists_and_reloads(tmp_path) -> None:
    path = tmp_path / "cache.json"
    KernelCache(path=path).set("GPU_A", "rope", "shape", "rope_hip")
    payload = json.loads(path.read_text())
    assert payload["version"] == CACHE_SCHEMA_VERSION == 2
    assert set(payload) == {"version", "entries"}
    assert KernelCache(path=path).get("GPU_A", "rope", "shape") == "rope_hip"


def test_reads_v1_schema(tmp_path) -> None:
    path = tmp_path / "cache.json"
    path.write_text(json.dumps({"GPU_A": {"rmsnorm": {"fp16_8x2048": "rmsnorm_triton"}}}))
    cache = KernelCache(path=path)
    assert cache.get("GPU_A", "rmsnorm", "fp16_8x2048") == "rmsnorm_triton"
    assert cache.get_record("GPU_A", "rmsnorm", "fp16_8x2048") == {"kernel": "rmsnorm_triton"}


def test_corrupt_file_is_kept_aside_and_logged(tmp_path, caplog) -> None:
    path = tmp_path / "cache.json"
    path.write_text("{not json")
    cache = KernelCache(path=path)
    assert cache.get("GPU_A", "rmsnorm", "shape") is None and len(cache) == 0
    assert "Unreadable kernel cache" in caplog.text
    assert (tmp_path / "cache.json.corrupt").read_text() == "{not json"
    cache.set("GPU_A", "rmsnorm", "shape", "rmsnorm_hip")
    assert KernelCache(path=path).get("GPU_A", "rmsnorm", "shape") == "rmsnorm_hip"
    assert not [f for f in tmp_path.iterdir() if f.name.endswith(".tmp")]


def test_stats_track_hit_rate(tmp_path) -> None:
    cache = KernelCache(path=tmp_path / "cache.json")
    cache.set("GPU_A", "rmsnorm", "shape", "rmsnorm_ref")
    cache.get("GPU_A", "rmsnorm", "shape")
    cache.get("GPU_A", "rmsnorm", "other")
    stats = cache.stats()
    assert (stats.hits, stats.misses, stats.hit_rate) == (1, 1, 0.5)
    assert stats.to_dict()["lookups"] == 2


def test_clear_and_env_override(tmp_path, monkeypatch) -> None:
    cache = KernelCache(path=tmp_path / "cache.json")
    cache.set("GPU_A", "rmsnorm", "shape", "rmsnorm_ref")
    cache.clear()
    assert len(cache) == 0
    assert KernelCache(path=tmp_path / "cache.json").get("GPU_A", "rmsnorm", "shape") is None
    monkeypatch.setenv("AKO_CACHE_PATH", str(tmp_path / "x" / "k.json"))
    assert default_cache_path() == tmp_path / "x" / "k.json"
