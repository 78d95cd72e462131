"""Per-operation latency measurement (wall clock and HIP events).

Semantics follow ``ako/benchmark/bench_op.py:30-472`` of the reference, since
the selector's decisions and every cache record are expressed in them:

* calls are timed in batches of ``inner`` calls sized to ~``TARGET_BATCH_MS``
  (synchronising around a single microsecond-scale call would time the
  synchronisation), and every statistic is per single call;
* ``latency_*`` is amortised wall clock (what a caller pays, launch included),
  ``gpu_p50_ms`` is device time from events recorded on the current stream;
  on ROCm ``torch.cuda.Event`` is a hipEvent;
* with ``flush_l2`` a scratch buffer is zeroed before every call and its
  calibrated cost is subtracted from both clocks.

MI355X difference: the flush is sized from the device rather than fixed at the
reference's 32 MiB. An MI355X has eight XCDs with 4 MB of L2 each; a memset
is spread over all of them, so evicting every L2 needs twice the aggregate
(64 MiB). The 256 MB Infinity Cache (MALL) is *not* evicted by this flush,
because zeroing more than 512 MB per call would swamp a microsecond kernel;
bandwidth roofline numbers therefore come from
``ako_amd.benchmark.roofline``, which rotates over input copies larger than
the MALL instead of flushing.
"""

from __future__ import annotations

import random
import statistics
import time
from dataclasses import dataclass
from functools import lru_cache
from typing import Any, Callable, Sequence

import torch

DTYPE_ALIASES: dict[str, torch.dtype] = {
    "fp16": torch.float16,
    "bf16": torch.bfloat16,
    "fp32": torch.float32,
}


def parse_dtypes(raw: Sequence[str]) -> list[torch.dtype]:
    """CLI dtype names (``fp16``/``bf16``/``fp32``) to torch dtypes."""
    unknown = [d for d in raw if d not in DTYPE_ALIASES]
    if unknown:
        raise ValueError(f"Unknown dtype(s) {unknown}; expected one of {sorted(DTYPE_ALIASES)}")
    return [DTYPE_ALIASES[d] for d in raw]


#: Work per timed batch, in ms.
TARGET_BATCH_MS = 1.0
MAX_INNER_ITERS = 200
#: Run-to-run coefficient of variation above which a number is flagged unstable.
UNSTABLE_CV = 0.10
#: The reference's flush size; the floor of the device-aware size below.
L2_FLUSH_BYTES = 32 * 1024 * 1024
#: XCDs per package on gfx942/gfx950 (the L2 reported by HIP is per XCD).
_XCDS = {"gfx942": 8, "gfx950": 8}


def _percentile(values: Sequence[float], p: float) -> float:
    """Index-truncated percentile (the reference's definition)."""
    if not values:
        return 0.0
    ordered = sorted(values)
    return ordered[min(int(len(ordered) * p), len(ordered) - 1)]


@dataclass(frozen=True)
class BenchResult:
    """Latency statistics of one kernel on one input, per single call."""

    kernel_name: str
    shape: tuple[int, ...]
    dtype: str
    device: str
    latency_p50_ms: float
    latency_p95_ms: float
    latency_mean_ms: float
    latency_std_ms: float
    samples_ms: list[float]
    gpu_p50_ms: float | None = None
    inner_iters: int = 1
    peak_memory_mb: float | None = None
    run_p50s: tuple[float, ...] = ()
    #: ``flushed``, ``off``, or ``n/a`` off the GPU.
    l2_state: str = "n/a"
    l2_flush_ms: float = 0.0
    graph_captured: int = 0

    @property
    def launch_overhead_ms(self) -> float | None:
        """Wall minus device time; deliberately not clamped at zero."""
        if self.gpu_p50_ms is None:
            return None
        return self.latency_p50_ms - self.gpu_p50_ms

    @property
    def _spread_samples(self) -> list[float]:
        return list(self.run_p50s) if len(self.run_p50s) > 1 else list(self.samples_ms)

    @property
    def median_ms(self) -> float:
        return statistics.median(self._spread_samples or [0.0])

    @property
    def iqr_ms(self) -> float:
        vals = self._spread_samples
        return _percentile(vals, 0.75) - _percentile(vals, 0.25)

    @property
    def cv(self) -> float:
        vals = self._spread_samples
        if len(vals) < 2:
            return 0.0
        mean = statistics.mean(vals)
        return statistics.stdev(vals) / mean if mean > 0 else 0.0

    @property
    def unstable(self) -> bool:
        return self.cv > UNSTABLE_CV

    def to_dict(self) -> dict[str, Any]:
        spread = self._spread_samples
        payload: dict[str, Any] = {
            "kernel_name": self.kernel_name,
            "shape": list(self.shape),
            "dtype": self.dtype,
            "device": self.device,
            "latency_p50_ms": round(self.latency_p50_ms, 4),
            "latency_p95_ms": round(self.latency_p95_ms, 4),
            "latency_mean_ms": round(self.latency_mean_ms, 4),
            "latency_std_ms": round(self.latency_std_ms, 4),
            "inner_iters": self.inner_iters,
            "runs": max(len(self.run_p50s), 1),
            "median_ms": round(self.median_ms, 4),
            "p25_ms": round(_percentile(spread, 0.25), 4),
            "p75_ms": round(_percentile(spread, 0.75), 4),
            "iqr_ms": round(self.iqr_ms, 4),
            "cv": round(self.cv, 4),
            "unstable": self.unstable,
            "l2_state": self.l2_state,
            "graph_captured": self.graph_captured,
            "samples_ms": [round(v, 7) for v in self.samples_ms],
        }
        if self.l2_flush_ms:
            payload["l2_flush_ms"] = round(self.l2_flush_ms, 4)
        if self.gpu_p50_ms is not None:
            payload["gpu_p50_ms"] = round(self.gpu_p50_ms, 4)
            payload["launch_overhead_ms"] = round(self.latency_p50_ms - self.gpu_p50_ms, 4)
        if self.peak_memory_mb is not None:
            payload["peak_memory_mb"] = round(self.peak_memory_mb, 2)
        return payload


def l2_flush_bytes(device: torch.device) -> int:
    """Bytes to zero so that every XCD's L2 is evicted (at least 32 MiB)."""
    if device.type != "cuda" or not torch.cuda.is_available():
        return L2_FLUSH_BYTES
    props = torch.cuda.get_device_properties(device)
    arch = str(getattr(props, "gcnArchName", "")).split(":")[0]
    l2 = int(getattr(props, "L2_cache_size", 0) or 0)
    return max(L2_FLUSH_BYTES, 2 * l2 * _XCDS.get(arch, 1))


@lru_cache(maxsize=None)
def _flush_buffer(device: torch.device) -> torch.Tensor:
    """One scratch buffer per device, alive for the whole process."""
    return torch.empty(l2_flush_bytes(device), dtype=torch.int8, device=device)


@lru_cache(maxsize=None)
def _flush_cost_ms(device: torch.device) -> tuple[float, float]:
    """(wall, device) cost of one flush, measured once through ``bench_op``."""
    result = bench_op(
        lambda b: b.zero_(),
        (_flush_buffer(device),),
        warmup=5,
        repeats=20,
        inner=10,
        flush_l2=False,
        kernel_name="l2_flush",
    )
    return result.latency_p50_ms, result.gpu_p50_ms or 0.0


def _calibrate_inner(
    fn: Callable[..., Any], args: tuple[Any, ...], kwargs: dict[str, Any], on_gpu: bool
) -> int:
    """Calls per timed batch so that one batch lasts about ``TARGET_BATCH_MS``."""
    if on_gpu:
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn(*args, **kwargs)
    if on_gpu:
        torch.cuda.synchronize()
    single_ms = (time.perf_counter() - t0) * 1e3
    if single_ms <= 0:
        return MAX_INNER_ITERS
    return max(1, min(MAX_INNER_ITERS, int(TARGET_BATCH_MS / single_ms)))


def bench_op(
    fn: Callable[..., Any],
    args: tuple[Any, ...],
    *,
    warmup: int = 10,
    repeats: int = 50,
    kernel_name: str = "unknown",
    call_kwargs: dict[str, Any] | None = None,
    inner: int | None = None,
    runs: int = 1,
    flush_l2: bool = True,
    graph: bool = False,
) -> BenchResult:
    """Time ``fn(*args, **call_kwargs)``; ``args[0]`` must be a tensor.

    ``runs`` > 1 repeats the whole measurement so the spread statistics
    describe run-to-run variability. ``graph`` captures ``fn`` in a HIP graph
    after warmup and replays it (falling back to eager timing, recorded as
    ``graph_captured=0``, when capture fails); the flush stays outside the graph.
    """
    x = args[0]
    if not isinstance(x, torch.Tensor):
        raise TypeError("bench_op needs a tensor as its first argument")
    kwargs = call_kwargs or {}
    on_gpu = x.is_cuda

    flush = _flush_buffer(x.device) if (flush_l2 and on_gpu) else None
    l2_state = "flushed" if flush is not None else ("off" if on_gpu else "n/a")
    flush_wall_ms, flush_gpu_ms = _flush_cost_ms(x.device) if flush is not None else (0.0, 0.0)

    for _ in range(warmup):
        fn(*args, **kwargs)
    if on_gpu:
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(x.device)

    timed: Callable[..., Any] = fn
    graph_captured = 0
    if graph and on_gpu:
        from ako_amd.benchmark.graph import try_capture

        captured = try_capture(fn, args, kwargs)
        if captured.captured and captured.replay is not None:
            replay = captured.replay

            def timed(*_a: Any, **_k: Any) -> None:
                replay()

            graph_captured = 1

    if inner is None:
        inner = _calibrate_inner(timed, args, kwargs, on_gpu)

    samples: list[float] = []
    gpu_samples: list[float] = []
    run_p50s: list[float] = []
    for _ in range(max(1, runs)):
        run_samples: list[float] = []
        for _ in range(repeats):
            if on_gpu:
                start = torch.cuda.Event(enable_timing=True)
                stop = torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                start.record()
                for _ in range(inner):
                    if flush is not None:
                        flush.zero_()
                    timed(*args, **kwargs)
                stop.record()
                torch.cuda.synchronize()
                wall_ms = (time.perf_counter() - t0) * 1e3
                gpu_samples.append(max(start.elapsed_time(stop) / inner - flush_gpu_ms, 0.0))
            else:
                t0 = time.perf_counter()
                for _ in range(inner):
                    timed(*args, **kwargs)
                wall_ms = (time.perf_counter() - t0) * 1e3
            run_samples.append(max(wall_ms / inner - flush_wall_ms, 0.0))
        run_p50s.append(_percentile(run_samples, 0.50))
        samples.extend(run_samples)

    peak_mb = torch.cuda.max_memory_allocated(x.device) / 1024**2 if on_gpu else None
    return BenchResult(
        kernel_name=kernel_name,
        shape=tuple(x.shape),
        dtype=str(x.dtype).replace("torch.", ""),
        device=str(x.device),
        latency_p50_ms=_percentile(samples, 0.50),
        latency_p95_ms=_percentile(samples, 0.95),
        latency_mean_ms=statistics.mean(samples),
        latency_std_ms=statistics.stdev(samples) if len(samples) > 1 else 0.0,
        samples_ms=samples,
        gpu_p50_ms=_percentile(gpu_samples, 0.50) if gpu_samples else None,
        inner_iters=inner,
        peak_memory_mb=peak_mb,
        run_p50s=tuple(run_p50s),
        l2_state=l2_state,
        l2_flush_ms=flush_wall_ms,
        graph_captured=graph_captured,
    )


def bootstrap_ci(
    values: Sequence[float], *, seed: int = 0, resamples: int = 1000, confidence: float = 0.95
) -> tuple[float, float]:
    """Seeded percentile-bootstrap interval of the median."""
    if not values:
        return (0.0, 0.0)
    rng = random.Random(seed)
    pool = list(values)
    medians = [statistics.median(rng.choices(pool, k=len(pool))) for _ in range(resamples)]
    tail = (1.0 - confidence) / 2
    return (_percentile(medians, tail), _percentile(medians, 1.0 - tail))


def bootstrap_ratio_ci(
    numerator: Sequence[float],
    denominator: Sequence[float],
    *,
    seed: int = 0,
    resamples: int = 2000,
    confidence: float = 0.95,
) -> tuple[float, float, float]:
    """``(median(num)/median(den), low, high)`` for two independent sample sets."""
    if not numerator or not denominator:
        raise ValueError("both sample sets must be non-empty")
    if min(denominator) <= 0:
        raise ValueError("denominator samples must be positive")
    rng = random.Random(seed)
    num, den = list(numerator), list(denominator)
    ratios = sorted(
        statistics.median(rng.choices(num, k=len(num)))
        / statistics.median(rng.choices(den, k=len(den)))
        for _ in range(resamples)
    )
    tail = (1.0 - confidence) / 2
    point = statistics.median(num) / statistics.median(den)
    return point, _percentile(ratios, tail), _percentile(ratios, 1.0 - tail)


def compare_paired(
    fn_a: Callable[..., Any],
    fn_b: Callable[..., Any],
    args: tuple[Any, ...],
    *,
    pairs: int = 11,
    seed: int = 0,
    warmup: int = 5,
    repeats: int = 20,
    call_kwargs: dict[str, Any] | None = None,
    inner: int | None = None,
    flush_l2: bool = True,
    graph: bool = False,
) -> dict[str, Any]:
    """A/B timing in alternation; ``speedup_median`` > 1 means ``fn_b`` is faster."""
    common = dict(
        warmup=warmup, repeats=repeats, call_kwargs=call_kwargs, inner=inner,
        flush_l2=flush_l2, graph=graph,
    )
    ratios: list[float] = []
    a_ms: list[float] = []
    b_ms: list[float] = []
    unstable = False
    captured = True
    for index in range(pairs):
        # Alternate who goes first so neither side always sees the warmer card.
        order = ((fn_a, "a"), (fn_b, "b")) if index % 2 == 0 else ((fn_b, "b"), (fn_a, "a"))
        got = {tag: bench_op(fn, args, kernel_name=tag, **common) for fn, tag in order}
        res_a, res_b = got["a"], got["b"]
        unstable = unstable or res_a.unstable or res_b.unstable
        captured = captured and bool(res_a.graph_captured) and bool(res_b.graph_captured)
        a_ms.append(res_a.latency_p50_ms)
        b_ms.append(res_b.latency_p50_ms)
        if res_b.latency_p50_ms > 0:
            ratios.append(res_a.latency_p50_ms / res_b.latency_p50_ms)
    low, high = bootstrap_ci(ratios, seed=seed)
    return {
        "pairs": len(ratios),
        "a_median_ms": round(statistics.median(a_ms), 4) if a_ms else 0.0,
        "b_median_ms": round(statistics.median(b_ms), 4) if b_ms else 0.0,
        "speedup_median": round(statistics.median(ratios), 4) if ratios else 0.0,
        "speedup_ci95": [round(low, 4), round(high, 4)],
        "significant": bool(ratios) and (low > 1.0 or high < 1.0),
        "unstable": unstable,
        "graph_captured": captured if graph else False,
    }


def bench_shapes(
    fn: Callable[..., Any],
    shapes: Sequence[tuple[int, ...]],
    *,
    dtype: torch.dtype = torch.float16,
    device: str = "cuda",
    weight_fn: Callable[[int], torch.Tensor] | None = None,
    warmup: int = 10,
    repeats: int = 30,
    kernel_name: str = "unknown",
) -> list[BenchResult]:
    """``bench_op`` over several ``(..., hidden)`` shapes with a ones weight."""
    results = []
    for shape in shapes:
        x = torch.randn(*shape, dtype=dtype, device=device)
        w = weight_fn(shape[-1]) if weight_fn else torch.ones(shape[-1], dtype=dtype, device=device)
        results.append(bench_op(fn, (x, w), warmup=warmup, repeats=repeats, kernel_name=kernel_name))
    return results
