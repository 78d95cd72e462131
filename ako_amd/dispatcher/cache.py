"""Persistent JSON cache of kernel-selection decisions.

The on-disk format is the reference's schema v2 (``ako/dispatcher/cache.py:3-21``),
kept byte-compatible so a cache file moves between the two implementations::

    {"version": 2,
     "entries": {"<gpu_key>": {"<op_name>": {"<shape_key>": {
         "kernel": "rmsnorm_hip", "created_at": "...", "latency_p50_ms": ...,
         "baseline_ms": ..., "speedup": ..., "best_baseline_ms": ...,
         "best_baseline_kernel": ..., "speedup_vs_best_baseline": ...,
         "max_error": ..., "error_budget": ..., "backend": "hip"}}}}}

Schema v1 (the document itself maps ``gpu -> op -> shape -> kernel name``) is
read and upgraded in memory (reference ``cache.py:103-108``). Saving writes a
pid-suffixed temporary file and renames it over the cache, so a crash never
leaves a truncated file; an unreadable file is logged, moved aside to
``<name>.corrupt`` and the cache starts empty (reference ``cache.py:86-101``).
The location defaults to ``~/.ako/kernel_cache.json`` and is overridden by
``AKO_CACHE_PATH``.
"""

from __future__ import annotations

import json
import logging
import os
from dataclasses import dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

CACHE_SCHEMA_VERSION = 2
DEFAULT_CACHE_PATH = Path.home() / ".ako" / "kernel_cache.json"

logger = logging.getLogger(__name__)


def default_cache_path() -> Path:
    override = os.environ.get("AKO_CACHE_PATH")
    return Path(override).expanduser() if override else DEFAULT_CACHE_PATH


@dataclass(frozen=True)
class CacheStats:
    """Lookup counters (the paper's cache hit-rate metric)."""

    hits: int = 0
    misses: int = 0

    @property
    def total(self) -> int:
        return self.hits + self.misses

    @property
    def hit_rate(self) -> float:
        return self.hits / self.total if self.total else 0.0

    def to_dict(self) -> dict[str, Any]:
        return {
            "hits": self.hits,
            "misses": self.misses,
            "lookups": self.total,
            "hit_rate": round(self.hit_rate, 4),
        }


class KernelCache:
    """``(gpu_key, op, shape_key) -> record`` decisions backed by one JSON file."""

    def __init__(self, path: Path | str | None = None, *, autosave: bool = True) -> None:
        self.path = Path(path) if path is not None else default_cache_path()
        self.autosave = autosave
        self._entries: dict[str, Any] = {}
        self._hits = 0
        self._misses = 0
        self.load()

    # -- persistence ---------------------------------------------------
    def load(self) -> None:
        self._entries = {}
        if not self.path.exists():
            return
        try:
            document = json.loads(self.path.read_text())
        except (json.JSONDecodeError, OSError) as exc:
            logger.warning("Unreadable kernel cache %s (%s); starting empty", self.path, exc)
            if isinstance(exc, json.JSONDecodeError):
                try:
                    os.replace(self.path, self.path.with_name(self.path.name + ".corrupt"))
                except OSError:
                    pass
            return
        self._entries = self._upgrade(document)

    @staticmethod
    def _upgrade(document: Any) -> dict[str, Any]:
        if not isinstance(document, dict):
            return {}
        if document.get("version") == CACHE_SCHEMA_VERSION:
            entries = document.get("entries", {})
            return entries if isinstance(entries, dict) else {}
        # v1: the top level is already gpu -> op -> shape -> "kernel_name".
        return {k: v for k, v in document.items() if k != "version" and isinstance(v, dict)}

    def save(self) -> None:
        self.path.parent.mkdir(parents=True, exist_ok=True)
        scratch = self.path.with_name(f".{self.path.name}.{os.getpid()}.tmp")
        scratch.write_text(
            json.dumps({"version": CACHE_SCHEMA_VERSION, "entries": self._entries}, indent=2)
        )
        os.replace(scratch, self.path)

    # -- lookups -------------------------------------------------------
    def get_record(self, gpu_key: str, op_name: str, shape_key: str) -> dict[str, Any] | None:
        """The stored record (a copy), or ``None`` on a miss."""
        value = self._entries.get(gpu_key, {}).get(op_name, {}).get(shape_key)
        if value is None:
            self._misses += 1
            return None
        self._hits += 1
        if isinstance(value, str):  # a v1 bare kernel name
            return {"kernel": value}
        return dict(value)

    def get(self, gpu_key: str, op_name: str, shape_key: str) -> str | None:
        record = self.get_record(gpu_key, op_name, shape_key)
        return None if record is None else record.get("kernel")

    def set(self, gpu_key: str, op_name: str, shape_key: str, kernel_name: str, **metrics: Any) -> None:
        """Store a decision with the metrics that justified it (``None`` values dropped)."""
        record: dict[str, Any] = {
            "kernel": kernel_name,
            "created_at": datetime.now(timezone.utc).isoformat(),
        }
        record.update((k, v) for k, v in metrics.items() if v is not None)
        self._entries.setdefault(gpu_key, {}).setdefault(op_name, {})[shape_key] = record
        if self.autosave:
            self.save()

    def clear(self) -> None:
        self._entries = {}
        self._hits = self._misses = 0
        if self.autosave:
            self.save()

    # -- introspection -------------------------------------------------
    def stats(self) -> CacheStats:
        return CacheStats(hits=self._hits, misses=self._misses)

    def to_dict(self) -> dict[str, Any]:
        return {"version": CACHE_SCHEMA_VERSION, "entries": dict(self._entries)}

    def __len__(self) -> int:
        return sum(len(shapes) for ops in self._entries.values() for shapes in ops.values())
