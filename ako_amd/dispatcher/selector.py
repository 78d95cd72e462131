"""Benchmark-driven kernel selection with a persistent decision cache.

The decision procedure is the reference's Algorithm 1
(``ako/dispatcher/selector.py:143-346``), kept step for step because the cache
records and the non-regression guarantee depend on it:

1. a process-local memo answers repeated calls of the same (op, shape, dtype,
   device, variant) without touching anything else;
2. otherwise the persistent cache is consulted for ``(gpu, op, shape_key)``;
3. on a miss, and only on a GPU (or with ``allow_cpu_tuning``), the reference
   kernel (the ``backend == "pytorch"`` entry) is run once for its output and
   timed; every other candidate is run, rejected if its max-abs error exceeds
   the dtype-aware budget (or raises), and timed otherwise;
4. the fastest survivor wins only if it beats the reference by ``min_speedup``;
   the decision and its metrics are written to the cache.

New here: every candidate's ulp report (``ako_amd.validation.ulp_report``) is
kept on the ``SelectionResult`` and serialised under ``ulp_reports``; the
cache record itself is unchanged.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Any

import torch

from ako_amd.benchmark.bench_op import bench_op
from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.hardware import get_device_info
from ako_amd.dispatcher.registry import KernelEntry, KernelFn, KernelRegistry, get_registry
from ako_amd.validation.numerical import (
    error_budget,
    error_in_ulps,
    max_abs_error_any,
    ulp_report,
)

#: Backends that count as baselines: what a user could already run without AKO.
BASELINE_BACKENDS = frozenset({"pytorch", "torch_native", "torch_compile"})


def _env_flag(name: str, default: bool = False) -> bool:
    raw = os.environ.get(name)
    if raw is None:
        return default
    return raw.strip().lower() in {"1", "true", "yes", "on"}


def shape_key(tensors: tuple[torch.Tensor, ...], extra: str | None = None) -> str:
    """Cache key of a call: ``"<shape0>_<dtype0>_<shape1>_..._<extra>"``.

    Example: ``(4, 1024, 16, 128)_float16_(1024, 64)_(1024, 64)_neox``.
    """
    if not tensors:
        raise ValueError("At least one tensor is required to build a shape key")
    first = tensors[0]
    parts = [str(tuple(first.shape)), str(first.dtype).replace("torch.", "")]
    parts += [str(tuple(t.shape)) for t in tensors[1:]]
    if extra:
        parts.append(extra)
    return "_".join(parts)


@dataclass(frozen=True)
class SelectionResult:
    """One selection decision (mirrors what the cache stores)."""

    op_name: str
    entry: KernelEntry
    shape_key: str
    #: ``cache``, ``benchmark``, ``default`` or ``forced``.
    source: str
    latency_p50_ms: float | None = None
    baseline_ms: float | None = None
    max_error: float | None = None
    candidates_evaluated: int = 0
    rejected: tuple[str, ...] = ()
    best_baseline_ms: float | None = None
    best_baseline_kernel: str | None = None
    ulp_reports: tuple[dict[str, Any], ...] = field(default=())
    #: Wall p50 (ms) of every candidate that was timed, reference included.
    latencies_ms: tuple[tuple[str, float], ...] = field(default=())

    @property
    def from_cache(self) -> bool:
        return self.source == "cache"

    @property
    def speedup(self) -> float | None:
        """Gain over the unfused reference (kept for continuity, not quotable)."""
        if self.baseline_ms and self.latency_p50_ms:
            return self.baseline_ms / self.latency_p50_ms
        return None

    @property
    def speedup_vs_best_baseline(self) -> float | None:
        """Gain over the fastest baseline: the number worth publishing."""
        if self.best_baseline_ms and self.latency_p50_ms:
            return self.best_baseline_ms / self.latency_p50_ms
        return None

    def to_dict(self) -> dict[str, Any]:
        speedup = self.speedup
        vs_best = self.speedup_vs_best_baseline
        return {
            "operation": self.op_name,
            "selected_kernel": self.entry.kernel_name,
            "backend": self.entry.backend,
            "shape_key": self.shape_key,
            "source": self.source,
            "from_cache": self.from_cache,
            "latency_p50_ms": self.latency_p50_ms,
            "baseline_ms": self.baseline_ms,
            "speedup": round(speedup, 3) if speedup else None,
            "best_baseline_ms": self.best_baseline_ms,
            "best_baseline_kernel": self.best_baseline_kernel,
            "speedup_vs_best_baseline": round(vs_best, 3) if vs_best else None,
            "max_error": self.max_error,
            "candidates_evaluated": self.candidates_evaluated,
            "rejected": list(self.rejected),
            "ulp_reports": [dict(r) for r in self.ulp_reports],
            "latencies_ms": dict(self.latencies_ms),
        }


class KernelSelector:
    """Chooses, per (device, op, shape, dtype), the fastest kernel that passes the gate."""

    def __init__(
        self,
        registry: KernelRegistry | None = None,
        cache: KernelCache | None = None,
        *,
        auto_tune: bool | None = None,
        error_threshold: float | None = None,
        min_speedup: float = 1.0,
        warmup: int = 5,
        repeats: int = 20,
        allow_cpu_tuning: bool = False,
    ) -> None:
        self.registry = get_registry() if registry is None else registry
        # Explicit None test: an empty KernelCache is falsy (it has __len__).
        self.cache = KernelCache() if cache is None else cache
        self.auto_tune = _env_flag("AKO_AUTOTUNE", True) if auto_tune is None else auto_tune
        self.allow_cpu_tuning = allow_cpu_tuning
        #: ``None``: derive the budget from dtype and magnitude (the gate).
        self.error_threshold = error_threshold
        self.min_speedup = min_speedup
        self.warmup = warmup
        self.repeats = repeats
        self._memo: dict[tuple[Any, ...], KernelFn] = {}

    # -- public API ----------------------------------------------------
    def select(
        self,
        op_name: str,
        x: torch.Tensor,
        *args: torch.Tensor,
        forced: str | None = None,
        extra_key: str | None = None,
        call_kwargs: dict[str, Any] | None = None,
    ) -> KernelFn:
        """The callable to run for this call; memoised on cheap hashables."""
        memo_key = (
            op_name,
            forced,
            extra_key,
            x.dtype,
            x.shape,
            x.device,
            tuple([a.shape for a in args]),
        )
        fn = self._memo.get(memo_key)
        if fn is None:
            fn = self.select_entry(
                op_name, x, *args, forced=forced, extra_key=extra_key, call_kwargs=call_kwargs
            ).entry.fn
            self._memo[memo_key] = fn
        return fn

    def clear_memo(self) -> None:
        self._memo.clear()

    def select_entry(
        self,
        op_name: str,
        x: torch.Tensor,
        *args: torch.Tensor,
        forced: str | None = None,
        extra_key: str | None = None,
        call_kwargs: dict[str, Any] | None = None,
    ) -> SelectionResult:
        """Like :meth:`select`, returning the whole decision record."""
        kernels = self.registry.list_kernels(op_name)
        if not kernels:
            raise ValueError(f"No kernels registered for op '{op_name}'")
        key = shape_key((x, *args), extra_key)

        if forced:
            entry = self.registry.get(op_name, forced)
            if entry is None:
                names = ", ".join(k.kernel_name for k in kernels)
                raise ValueError(f"Unknown kernel '{forced}' for op '{op_name}' (available: {names})")
            return SelectionResult(op_name, entry, key, source="forced")

        gpu_key = get_device_info(x.device).cache_key
        record = self.cache.get_record(gpu_key, op_name, key)
        if record:
            entry = self.registry.get(op_name, record["kernel"])
            if entry is not None:
                return SelectionResult(
                    op_name,
                    entry,
                    key,
                    source="cache",
                    latency_p50_ms=record.get("latency_p50_ms"),
                    baseline_ms=record.get("baseline_ms"),
                    max_error=record.get("max_error"),
                    best_baseline_ms=record.get("best_baseline_ms"),
                    best_baseline_kernel=record.get("best_baseline_kernel"),
                )

        tunable = x.device.type == "cuda" or self.allow_cpu_tuning
        if not self.auto_tune or not tunable or len(kernels) == 1:
            default = self.registry.default(op_name)
            assert default is not None
            return SelectionResult(op_name, default, key, source="default")

        return self._benchmark_and_select(
            op_name, kernels, (x, *args), key=key, call_kwargs=call_kwargs or {}, gpu_key=gpu_key
        )

    # -- autotuning ----------------------------------------------------
    def _time(self, entry: KernelEntry, tensors: tuple[torch.Tensor, ...], kwargs: dict[str, Any]) -> float:
        result = bench_op(
            entry.fn,
            tensors,
            warmup=self.warmup,
            repeats=self.repeats,
            kernel_name=entry.kernel_name,
            call_kwargs=kwargs,
        )
        return result.latency_p50_ms

    def _benchmark_and_select(
        self,
        op_name: str,
        kernels: list[KernelEntry],
        tensors: tuple[torch.Tensor, ...],
        *,
        key: str,
        call_kwargs: dict[str, Any],
        gpu_key: str,
    ) -> SelectionResult:
        reference = next((k for k in kernels if k.backend == "pytorch"), kernels[-1])
        ref_out = reference.fn(*tensors, **call_kwargs)
        reference_ms = self._time(reference, tensors, call_kwargs)
        budget = error_budget(ref_out) if self.error_threshold is None else self.error_threshold

        winner, winner_ms, winner_err = reference, reference_ms, 0.0
        evaluated = 1
        rejected: list[str] = []
        reports: list[dict[str, Any]] = []
        baseline_ms: dict[str, float] = {reference.kernel_name: reference_ms}
        timed: dict[str, float] = {reference.kernel_name: reference_ms}

        for entry in kernels:
            if entry.kernel_name == reference.kernel_name:
                continue
            try:
                out = entry.fn(*tensors, **call_kwargs)
                err = max_abs_error_any(ref_out, out)
                report = ulp_report(ref_out, out, kernel=entry.kernel_name)
                report["error_budget"] = budget
                report["passed"] = err <= budget
                reports.append(report)
                if err > budget:
                    rejected.append(
                        f"{entry.kernel_name}: max_error={err:.3e} > budget={budget:.3e} "
                        f"({error_in_ulps(ref_out, out):.1f} ulps)"
                    )
                    continue
                latency = self._time(entry, tensors, call_kwargs)
            except Exception as exc:  # a broken candidate never breaks dispatch
                rejected.append(f"{entry.kernel_name}: {type(exc).__name__}: {exc}")
                continue
            evaluated += 1
            timed[entry.kernel_name] = latency
            if entry.backend in BASELINE_BACKENDS:
                baseline_ms[entry.kernel_name] = latency
            if latency < winner_ms and reference_ms >= latency * self.min_speedup:
                winner, winner_ms, winner_err = entry, latency, err

        best_baseline = min(baseline_ms, key=baseline_ms.__getitem__)
        best_baseline_ms = baseline_ms[best_baseline]
        self.cache.set(
            gpu_key,
            op_name,
            key,
            winner.kernel_name,
            latency_p50_ms=round(winner_ms, 4),
            baseline_ms=round(reference_ms, 4),
            speedup=round(reference_ms / winner_ms, 3) if winner_ms > 0 else None,
            best_baseline_ms=round(best_baseline_ms, 4),
            best_baseline_kernel=best_baseline,
            speedup_vs_best_baseline=(
                round(best_baseline_ms / winner_ms, 3) if winner_ms > 0 else None
            ),
            max_error=winner_err,
            error_budget=budget,
            backend=winner.backend,
        )
        return SelectionResult(
            op_name,
            winner,
            key,
            source="benchmark",
            latency_p50_ms=winner_ms,
            baseline_ms=reference_ms,
            max_error=winner_err,
            candidates_evaluated=evaluated,
            rejected=tuple(rejected),
            best_baseline_ms=best_baseline_ms,
            best_baseline_kernel=best_baseline,
            ulp_reports=tuple(reports),
            latencies_ms=tuple(timed.items()),
        )


_GLOBAL_SELECTOR: KernelSelector | None = None


def get_selector() -> KernelSelector:
    """The process-wide selector behind every public ``ako_amd`` operation."""
    global _GLOBAL_SELECTOR
    if _GLOBAL_SELECTOR is None:
        _GLOBAL_SELECTOR = KernelSelector()
    return _GLOBAL_SELECTOR


def reset_selector() -> None:
    """Drop the process-wide selector (tests, CLI overrides)."""
    global _GLOBAL_SELECTOR
    _GLOBAL_SELECTOR = None
