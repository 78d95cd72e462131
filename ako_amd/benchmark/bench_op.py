"""Per-operation latency measurement for kernel selection, MI355X-first.

A selection needs, for every candidate on the same input, the per-call cost a
caller pays (host wall clock, launch included) and the device time. Both clocks
time *batches* of calls: synchronising around one microsecond-scale call would
time the synchronisation. Every figure reported is per single call. The record
layout (``BenchResult.to_dict``) is the reference's
(``ako/benchmark/bench_op.py:30-145``), because cache records and reports are
written in it.

**Cold inputs by rotation, not by flushing.** An MI355X keeps 4 MiB of L2 in
each of its 8 XCDs and a 256 MiB Infinity Cache (MALL) in front of HBM. A flush
that evicted both would write more than half a gigabyte per call, hundreds of
microseconds around a kernel of a few, and subtracting its calibrated cost back
out adds the flush's own jitter to every sample. Here the call's tensor
arguments are instead replicated into a ring of copies, and consecutive calls
read consecutive copies. When the ring holds at least 2 x (L2 + MALL) bytes,
every call reads inputs that at least that much traffic has passed over since
they were last touched: cold, with nothing added to the timed region and
nothing subtracted. Inputs that large on their own need no copies. Very small
inputs would need tens of thousands of copies, so the ring is capped at
``MAX_RING_COPIES`` (and at a quarter of the free device memory);
``l2_state`` then records what the ring does reach (``"cold"``,
``"l2-cold"`` when it covers only the L2s, or ``"warm"``).

Graph mode captures one pass over (up to ``GRAPH_RING_CALLS`` entries of) the
ring into a single HIP graph and times replays, which removes the host launch
cost from the wall clock as well.
"""

from __future__ import annotations

import math
import statistics
import time
from dataclasses import dataclass, field
from functools import lru_cache
from typing import Any, Callable, Sequence

import numpy as np
import torch

DTYPE_ALIASES: dict[str, torch.dtype] = {
    "fp16": torch.float16,
    "bf16": torch.bfloat16,
    "fp32": torch.float32,
}


def parse_dtypes(raw: Sequence[str]) -> list[torch.dtype]:
    """CLI dtype names (``fp16``/``bf16``/``fp32``) to torch dtypes."""
    bad = sorted(set(raw) - set(DTYPE_ALIASES))
    if bad:
        raise ValueError(f"Unknown dtype(s) {bad}; expected one of {sorted(DTYPE_ALIASES)}")
    return [DTYPE_ALIASES[name] for name in raw]


#: Device (or host) time one timed batch should last, in ms.
TARGET_BATCH_MS = 1.0
MAX_INNER_ITERS = 200
#: Coefficient of variation of the run medians above which a result is unstable.
UNSTABLE_CV = 0.10
#: Largest number of input copies in a rotation ring.
MAX_RING_COPIES = 1024
#: Ring entries one captured graph walks through.
GRAPH_RING_CALLS = 16

#: Last-level cache in front of HBM, per ISA (not reported by HIP).
_MALL_BYTES = {"gfx950": 256 << 20, "gfx942": 256 << 20}
#: XCDs per package; HIP's L2 size is per XCD.
_XCDS = {"gfx950": 8, "gfx942": 8}


@lru_cache(maxsize=None)
def cache_bytes(device: torch.device) -> tuple[int, int]:
    """``(all L2s, MALL)`` in bytes of a GPU; ``(0, 0)`` elsewhere."""
    if device.type != "cuda" or not torch.cuda.is_available():
        return 0, 0
    props = torch.cuda.get_device_properties(device)
    isa = str(getattr(props, "gcnArchName", "")).split(":")[0]
    l2 = int(getattr(props, "L2_cache_size", 0) or 0) * _XCDS.get(isa, 1)
    return l2, _MALL_BYTES.get(isa, 0)


def percentile(values: Sequence[float], q: float) -> float:
    """Nearest-rank percentile: the smallest value with at least ``q`` of the
    samples at or below it (0.0 for no samples)."""
    if not values:
        return 0.0
    ordered = sorted(values)
    rank = max(1, math.ceil(q * len(ordered)))
    return ordered[min(rank, len(ordered)) - 1]


@dataclass(frozen=True)
class BenchResult:
    """Latency statistics of one kernel on one input, per single call.

    ``latency_*`` is amortised wall clock (what a caller pays); ``gpu_p50_ms``
    is device time from hipEvents on the current stream. ``run_p50s`` holds the
    median of each independent run; the spread statistics use them when there
    are several runs, else the batch samples.
    """

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
    #: ``"cold"``, ``"l2-cold"``, ``"warm"`` on a GPU; ``"n/a"`` on the host.
    l2_state: str = "n/a"
    #: Per-call cost subtracted from the clocks; always 0 with input rotation.
    l2_flush_ms: float = 0.0
    graph_captured: int = 0
    #: Copies of the inputs the calls rotated over (1: the caller's own).
    input_copies: int = 1
    _spread: tuple[float, ...] = field(default=(), init=False, repr=False, compare=False)

    def __post_init__(self) -> None:
        spread = self.run_p50s if len(self.run_p50s) > 1 else tuple(self.samples_ms)
        object.__setattr__(self, "_spread", tuple(spread))

    @property
    def launch_overhead_ms(self) -> float | None:
        """Wall minus device time (negative values are kept: they show noise)."""
        return None if self.gpu_p50_ms is None else self.latency_p50_ms - self.gpu_p50_ms

    @property
    def median_ms(self) -> float:
        return statistics.median(self._spread) if self._spread else 0.0

    @property
    def iqr_ms(self) -> float:
        return percentile(self._spread, 0.75) - percentile(self._spread, 0.25)

    @property
    def cv(self) -> float:
        if len(self._spread) < 2:
            return 0.0
        mean = statistics.fmean(self._spread)
        return statistics.stdev(self._spread) / mean if mean > 0 else 0.0

    @property
    def unstable(self) -> bool:
        return self.cv > UNSTABLE_CV

    def to_dict(self) -> dict[str, Any]:
        def r4(v: float) -> float:
            return round(v, 4)

        out: dict[str, Any] = {
            "kernel_name": self.kernel_name,
            "shape": list(self.shape),
            "dtype": self.dtype,
            "device": self.device,
            "latency_p50_ms": r4(self.latency_p50_ms),
            "latency_p95_ms": r4(self.latency_p95_ms),
            "latency_mean_ms": r4(self.latency_mean_ms),
            "latency_std_ms": r4(self.latency_std_ms),
            "inner_iters": self.inner_iters,
            "runs": max(1, len(self.run_p50s)),
            "median_ms": r4(self.median_ms),
            "p25_ms": r4(percentile(self._spread, 0.25)),
            "p75_ms": r4(percentile(self._spread, 0.75)),
            "iqr_ms": r4(self.iqr_ms),
            "cv": r4(self.cv),
            "unstable": self.unstable,
            "l2_state": self.l2_state,
            "graph_captured": self.graph_captured,
            "input_copies": self.input_copies,
            "samples_ms": [round(v, 7) for v in self.samples_ms],
        }
        if self.l2_flush_ms:
            out["l2_flush_ms"] = r4(self.l2_flush_ms)
        if self.gpu_p50_ms is not None:
            out["gpu_p50_ms"] = r4(self.gpu_p50_ms)
            out["launch_overhead_ms"] = r4(self.latency_p50_ms - self.gpu_p50_ms)
        if self.peak_memory_mb is not None:
            out["peak_memory_mb"] = round(self.peak_memory_mb, 2)
        return out


class InputRing:
    """Argument tuples that successive calls cycle through.

    Entry 0 is the caller's own arguments; the other entries hold copies of
    every contiguous tensor argument. Non-tensors, and tensors whose strided
    layout a copy would not keep, are shared by all entries (``shared`` counts
    the latter). Each tensor's copies live in one slab allocated by a single
    broadcast copy, and the per-entry views are made once, so taking the next
    entry costs a list index.
    """

    def __init__(self, args: tuple[Any, ...], copies: int) -> None:
        copies = max(1, int(copies))
        self.copies = copies
        self.shared = 0
        slabs: list[Any] = []
        for a in args:
            if isinstance(a, torch.Tensor) and copies > 1 and a.is_contiguous():
                slabs.append(a.unsqueeze(0).expand(copies - 1, *a.shape).clone())
            else:
                self.shared += int(isinstance(a, torch.Tensor) and copies > 1)
                slabs.append(None)
        self.entries: list[tuple[Any, ...]] = [tuple(args)]
        for i in range(copies - 1):
            self.entries.append(tuple(a if s is None else s[i] for a, s in zip(args, slabs)))
        self._next = 0

    def __len__(self) -> int:
        return self.copies

    def next(self) -> tuple[Any, ...]:
        entry = self.entries[self._next]
        self._next = (self._next + 1) % self.copies
        return entry


def _tensor_bytes(args: tuple[Any, ...]) -> int:
    return sum(a.numel() * a.element_size() for a in args if isinstance(a, torch.Tensor))


#: Share of the device's free memory a ring may take (first-sight selection in
#: a serving process must not be the allocation that runs it out of memory).
RING_FREE_SHARE = 0.25


def plan_ring(args: tuple[Any, ...], device: torch.device, cold: bool) -> tuple[int, str]:
    """``(copies, l2_state)`` of the rotation that makes calls read cold inputs.

    The ring wants 2 x (L2 + MALL) bytes, holds at most ``MAX_RING_COPIES``
    copies and never more than ``RING_FREE_SHARE`` of the free device memory;
    ``l2_state`` says what the ring it gets can reach.
    """
    l2, mall = cache_bytes(device)
    if device.type != "cuda":
        return 1, "n/a"
    if not cold:
        return 1, "warm"
    per_call = max(1, _tensor_bytes(args))
    want = 2 * (l2 + mall)
    copies = min(MAX_RING_COPIES, max(1, math.ceil(want / per_call)))
    if copies > 1:
        free, _ = torch.cuda.mem_get_info(device)
        copies = max(1, min(copies, int(RING_FREE_SHARE * free) // per_call))
    return copies, ring_state(copies * per_call, l2, mall)


def ring_state(ring_bytes: int, l2: int, mall: int) -> str:
    if ring_bytes >= 2 * (l2 + mall):
        return "cold"
    if l2 and ring_bytes >= 2 * l2:
        return "l2-cold"
    return "warm"


def _sync(on_gpu: bool) -> None:
    if on_gpu:
        torch.cuda.synchronize()


def _batch(run: Callable[[], None], calls: int, on_gpu: bool) -> tuple[float, float | None]:
    """Wall and device ms of ``calls`` invocations of ``run`` (device: None on the host)."""
    if not on_gpu:
        t0 = time.perf_counter()
        for _ in range(calls):
            run()
        return (time.perf_counter() - t0) * 1e3, None
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    begin.record()
    for _ in range(calls):
        run()
    end.record()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3, begin.elapsed_time(end)


def _make_runner(fn: Callable[..., Any], ring: InputRing, kwargs: dict[str, Any], on_gpu: bool,
                 graph: bool) -> tuple[Callable[[], None], int, int, InputRing]:
    """``(run, calls per run, graph_captured, ring actually used)``.

    Eagerly a run is one call on the next ring entry. With ``graph`` a run is
    one replay of a graph holding one call per entry of a (possibly shorter)
    ring; if capture fails the eager runner is returned instead.
    """
    def eager() -> None:
        fn(*ring.next(), **kwargs)

    if not (graph and on_gpu):
        return eager, 1, 0, ring
    from ako_amd.benchmark.graph import capture_calls

    entries = ring.entries[:GRAPH_RING_CALLS]
    captured = capture_calls(fn, entries, kwargs)
    if captured.graph is None:
        return eager, 1, 0, ring
    return captured.replay, len(entries), 1, ring


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
    cold: bool = True,
    graph: bool = False,
) -> BenchResult:
    """Time ``fn(*args, **call_kwargs)``; ``args[0]`` must be a tensor.

    ``repeats`` timed batches of ``inner`` calls each (``inner`` chosen so that
    a batch lasts about ``TARGET_BATCH_MS`` unless given), repeated ``runs``
    times so that the spread describes run-to-run variation. ``cold`` rotates
    over input copies on a GPU (see the module docstring). ``graph`` replays a
    captured HIP graph instead of launching from the host.
    """
    x = args[0]
    if not isinstance(x, torch.Tensor):
        raise TypeError("bench_op needs a tensor as its first argument")
    kwargs = dict(call_kwargs or {})
    on_gpu = x.is_cuda
    copies, state = plan_ring(args, x.device, cold)
    ring = InputRing(args, copies)
    if ring.shared:
        state = "warm"  # a strided input is re-read by every call

    for _ in range(max(warmup, 1 if graph else 0)):
        fn(*ring.next(), **kwargs)
    _sync(on_gpu)
    if on_gpu:
        torch.cuda.reset_peak_memory_stats(x.device)

    run, per_run, captured, ring = _make_runner(fn, ring, kwargs, on_gpu, graph)
    if captured and not ring.shared:
        # The graph walks only its own entries: the state is what they cover.
        l2, mall = cache_bytes(x.device)
        state = ring_state(per_run * _tensor_bytes(args), l2, mall) if cold else "warm"

    if inner is None:
        probe_wall, probe_dev = _batch(run, 2, on_gpu)
        single = (probe_dev if probe_dev else probe_wall) / (2 * per_run)
        inner = MAX_INNER_ITERS if single <= 0 else int(min(MAX_INNER_ITERS, max(1, TARGET_BATCH_MS / single)))
    batches = max(1, math.ceil(inner / per_run))
    calls = batches * per_run

    wall: list[float] = []
    device: list[float] = []
    run_p50s: list[float] = []
    for _ in range(max(1, runs)):
        this_run: list[float] = []
        for _ in range(repeats):
            w, d = _batch(run, batches, on_gpu)
            this_run.append(w / calls)
            if d is not None:
                device.append(d / calls)
        run_p50s.append(percentile(this_run, 0.5))
        wall.extend(this_run)

    return BenchResult(
        kernel_name=kernel_name,
        shape=tuple(x.shape),
        dtype=str(x.dtype).removeprefix("torch."),
        device=str(x.device),
        latency_p50_ms=percentile(wall, 0.5),
        latency_p95_ms=percentile(wall, 0.95),
        latency_mean_ms=statistics.fmean(wall),
        latency_std_ms=statistics.stdev(wall) if len(wall) > 1 else 0.0,
        samples_ms=wall,
        gpu_p50_ms=percentile(device, 0.5) if device else None,
        inner_iters=calls,
        peak_memory_mb=torch.cuda.max_memory_allocated(x.device) / 2**20 if on_gpu else None,
        run_p50s=tuple(run_p50s),
        l2_state=state,
        graph_captured=captured,
        input_copies=len(ring),
    )


# -- statistics ------------------------------------------------------------------


def bootstrap_ci(values: Sequence[float], *, seed: int = 0, resamples: int = 1000,
                 confidence: float = 0.95) -> tuple[float, float]:
    """Seeded percentile-bootstrap interval of the median of ``values``."""
    if not values:
        return 0.0, 0.0
    rng = np.random.default_rng(seed)
    data = np.asarray(values, dtype=np.float64)
    medians = np.median(rng.choice(data, size=(resamples, data.size), replace=True), axis=1)
    alpha = (1.0 - confidence) / 2
    low, high = np.quantile(medians, [alpha, 1.0 - alpha])
    return float(low), float(high)


def bootstrap_ratio_ci(numerator: Sequence[float], denominator: Sequence[float], *, seed: int = 0,
                       resamples: int = 2000, confidence: float = 0.95) -> tuple[float, float, float]:
    """``(median(num) / median(den), low, high)`` for two independent samples."""
    if not numerator or not denominator:
        raise ValueError("both sample sets must be non-empty")
    num = np.asarray(numerator, dtype=np.float64)
    den = np.asarray(denominator, dtype=np.float64)
    if den.min() <= 0:
        raise ValueError("denominator samples must be positive")
    rng = np.random.default_rng(seed)
    ratios = (np.median(rng.choice(num, size=(resamples, num.size)), axis=1)
              / np.median(rng.choice(den, size=(resamples, den.size)), axis=1))
    alpha = (1.0 - confidence) / 2
    low, high = np.quantile(ratios, [alpha, 1.0 - alpha])
    return float(np.median(num) / np.median(den)), float(low), float(high)


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
    cold: bool = True,
    graph: bool = False,
) -> dict[str, Any]:
    """A/B timing on the same inputs; ``speedup_median`` > 1 means ``fn_b`` is faster.

    Each of the ``pairs`` rounds times ``repeats`` batches in the order A B B A
    (repeated), so that a clock or thermal drift within the round adds equally
    to both sides, and the round's ratio is total A time over total B time.
    The interval is a bootstrap over rounds.
    """
    x = args[0]
    if not isinstance(x, torch.Tensor):
        raise TypeError("compare_paired needs a tensor as its first argument")
    kwargs = dict(call_kwargs or {})
    on_gpu = x.is_cuda
    copies, _ = plan_ring(args, x.device, cold)
    ring = InputRing(args, copies)
    for fn in (fn_a, fn_b):
        for _ in range(max(warmup, 1)):
            fn(*ring.next(), **kwargs)
    _sync(on_gpu)
    run_a, per_a, cap_a, _ = _make_runner(fn_a, ring, kwargs, on_gpu, graph)
    run_b, per_b, cap_b, _ = _make_runner(fn_b, ring, kwargs, on_gpu, graph)
    if inner is None:
        w, d = _batch(run_a, 2, on_gpu)
        single = (d if d else w) / (2 * per_a)
        inner = MAX_INNER_ITERS if single <= 0 else int(min(MAX_INNER_ITERS, max(1, TARGET_BATCH_MS / single)))
    n_a, n_b = max(1, math.ceil(inner / per_a)), max(1, math.ceil(inner / per_b))

    def per_call(run, n, per):
        wall_ms, _ = _batch(run, n, on_gpu)  # what a caller pays, as latency_p50_ms
        return wall_ms / (n * per)

    ratios, a_ms, b_ms = [], [], []
    unstable = False
    for _ in range(max(1, pairs)):
        ta: list[float] = []
        tb: list[float] = []
        for i in range(max(1, repeats)):
            order = ((run_a, n_a, per_a, ta), (run_b, n_b, per_b, tb))
            if i % 2:
                order = order[::-1]
            for run, n, per, sink in order:
                sink.append(per_call(run, n, per))
        a, b = statistics.median(ta), statistics.median(tb)
        for side in (ta, tb):
            if len(side) > 1 and statistics.fmean(side) > 0:
                unstable = unstable or statistics.stdev(side) / statistics.fmean(side) > UNSTABLE_CV
        a_ms.append(a)
        b_ms.append(b)
        if b > 0:
            ratios.append(sum(ta) / sum(tb))
    low, high = bootstrap_ci(ratios, seed=seed)
    return {
        "pairs": len(ratios),
        "a_median_ms": round(statistics.median(a_ms), 4),
        "b_median_ms": round(statistics.median(b_ms), 4),
        "speedup_median": round(statistics.median(ratios), 4) if ratios else 0.0,
        "speedup_ci95": [round(low, 4), round(high, 4)],
        "significant": bool(ratios) and (low > 1.0 or high < 1.0),
        "unstable": unstable,
        "graph_captured": bool(cap_a and cap_b) if graph else False,
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
    seed: int = 0,
) -> list[BenchResult]:
    """``bench_op`` of ``fn(x, w)`` over ``(..., hidden)`` shapes: x ~ N(0, 1)
    from a seeded generator, w from ``weight_fn(hidden)`` or ones."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for shape in shapes:
        x = torch.randn(*shape, generator=gen).to(device=device, dtype=dtype)
        w = weight_fn(shape[-1]) if weight_fn else torch.ones(shape[-1], dtype=dtype, device=device)
        out.append(bench_op(fn, (x, w), warmup=warmup, repeats=repeats, kernel_name=kernel_name))
    return out
