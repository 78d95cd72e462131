"""HBM roofline accounting for the streaming kernels.

The four operations do O(1) flops per byte, so their bound is HBM bandwidth
(MFMA is deliberately unused). ``alg_bytes_*`` give the bytes a perfect
kernel must move per call (every input read once, every output written
once); achieved bandwidth is that figure over the measured device time.

Device time comes from HIP events recorded on the stream the kernels are
launched on (the HIP candidates launch on torch's current stream, so
``torch.cuda.Event`` records land on the same stream). To keep a
measurement cold without a per-call flush, callers cycle through input sets
whose total size exceeds twice the MI355X's Infinity Cache (256 MB) plus its
L2s (``copies_for_cold``), so no launch finds its inputs cached.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass, field
from typing import Any, Callable, Sequence

import torch

#: Published peak HBM bandwidth per ISA, GB/s (MI355X/MI350X: 8 TB/s HBM3E;
#: MI300X/MI325X: 5.3/6.0 TB/s; the gfx942 figure is the MI300X one).
HBM_PEAK_GBPS = {"gfx950": 8000.0, "gfx942": 5300.0}
#: Infinity Cache (MALL) + aggregate L2 per ISA, bytes: what a cold
#: measurement must exceed.
CACHE_BYTES = {"gfx950": 256 * 2**20 + 8 * 4 * 2**20, "gfx942": 256 * 2**20 + 8 * 4 * 2**20}


def elem_bytes(dtype: torch.dtype) -> int:
    return torch.finfo(dtype).bits // 8


def alg_bytes_rmsnorm(rows: int, hidden: int, dtype: torch.dtype, w_dtype: torch.dtype | None = None) -> int:
    b = elem_bytes(dtype)
    return 2 * rows * hidden * b + hidden * elem_bytes(w_dtype or dtype)


def alg_bytes_rmsnorm_residual(rows: int, hidden: int, dtype: torch.dtype,
                               w_dtype: torch.dtype | None = None) -> int:
    b = elem_bytes(dtype)
    return 4 * rows * hidden * b + hidden * elem_bytes(w_dtype or dtype)


def alg_bytes_rope(batch: int, seq: int, heads: int, head_dim: int, dtype: torch.dtype,
                   table_dtype: torch.dtype) -> int:
    return 2 * batch * seq * heads * head_dim * elem_bytes(dtype) + 2 * seq * (head_dim // 2) * elem_bytes(table_dtype)


def alg_bytes_rope_qk_cache(batch: int, seq: int, q_heads: int, kv_heads: int, head_dim: int,
                            dtype: torch.dtype, table_dtype: torch.dtype, *, values: bool = True) -> int:
    """q read and written, k read and written into the cache, v (when given)
    read and copied into the cache, one table row pair per token."""
    heads = q_heads + kv_heads + (kv_heads if values else 0)
    return 2 * batch * seq * heads * head_dim * elem_bytes(dtype) + 2 * seq * (head_dim // 2) * elem_bytes(table_dtype)


def alg_bytes_rmsnorm_shard_partial(rows: int, shard: int, dtype: torch.dtype, *, residual: bool) -> int:
    """x (and r) read, s written with a residual; one fp32 partial sum per row."""
    return (3 if residual else 1) * rows * shard * elem_bytes(dtype) + 4 * rows


def alg_bytes_rmsnorm_shard_apply(rows: int, shard: int, dtype: torch.dtype) -> int:
    """s read, y written, the weight slice and one fp32 total per row read."""
    return 2 * rows * shard * elem_bytes(dtype) + shard * elem_bytes(dtype) + 4 * rows


def alg_bytes_swiglu(rows: int, n: int, dtype: torch.dtype) -> int:
    return 3 * rows * n * elem_bytes(dtype)


def device_arch(device: torch.device | None = None) -> str | None:
    if not torch.cuda.is_available():
        return None
    props = torch.cuda.get_device_properties(device or torch.cuda.current_device())
    return str(getattr(props, "gcnArchName", "")).split(":")[0] or None


def hbm_peak_gbps(device: torch.device | None = None) -> float:
    """Published peak of this device's ISA (MI355X figure when unknown)."""
    return HBM_PEAK_GBPS.get(device_arch(device) or "", HBM_PEAK_GBPS["gfx950"])


def copies_for_cold(bytes_per_set: int, device: torch.device | None = None, minimum: int = 2) -> int:
    """Input sets to rotate through so the cycle exceeds twice MALL + L2."""
    cache = CACHE_BYTES.get(device_arch(device) or "", CACHE_BYTES["gfx950"])
    need = -(-2 * cache // max(bytes_per_set, 1))
    return max(minimum, int(need))


@dataclass
class LaunchStats:
    """Per-launch device durations of one kernel configuration."""

    name: str
    alg_bytes: int
    durations_ms: list[float] = field(default_factory=list)

    @property
    def mean_ms(self) -> float:
        return statistics.fmean(self.durations_ms) if self.durations_ms else 0.0

    @property
    def p50_ms(self) -> float:
        return statistics.median(self.durations_ms) if self.durations_ms else 0.0

    def gbps(self, which: str = "mean") -> float:
        ms = self.mean_ms if which == "mean" else self.p50_ms
        return self.alg_bytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0

    def to_dict(self, peak_gbps: float) -> dict[str, Any]:
        return {
            "name": self.name,
            "alg_bytes": self.alg_bytes,
            "launches": len(self.durations_ms),
            "mean_us": round(self.mean_ms * 1e3, 3),
            "p50_us": round(self.p50_ms * 1e3, 3),
            "gbps": round(self.gbps(), 1),
            "pct_hbm_peak": round(100.0 * self.gbps() / peak_gbps, 2),
        }


# Spin cycles queued ahead of a timed region (torch's clock-bounded spin
# kernel, one wavefront, no memory traffic): 200k cycles are 80-140 us at the
# clocks MI355X runs, longer than the host needs to queue the first timed
# event and launch behind it.
_LEAD_CYCLES = 200_000


def queue_lead() -> None:
    """Keep the device busy while the host queues a timed region. Recorded on
    an idle device, the region's first event completes at once, and the
    host's time to submit the first launch behind it is counted as device
    time (a few to tens of microseconds, seen as an outlier on the first of a
    run of per-launch timings). With this spin queued first, the first event
    is reached with the first timed launch already queued behind it."""
    torch.cuda._sleep(_LEAD_CYCLES)


def time_steps(calls: Sequence[tuple[str, int, Callable[[], Any]]], *, steps: int) -> float:
    """Milliseconds for ``steps`` back-to-back passes over ``calls``, bracketed by
    one pair of events (no per-launch events inside, so nothing but the
    kernels and their launches is timed)."""
    stream = torch.cuda.current_stream()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    begin.record(stream)
    for _ in range(steps):
        for _, _, fn in calls:
            fn()
    end.record(stream)
    torch.cuda.synchronize()
    return begin.elapsed_time(end)


#: Untimed passes that ``time_each_launch`` queues ahead of its timed ones.
LEAD_PASSES = 3


def time_each_launch(
    calls: Sequence[tuple[str, int, Callable[[], Any]]], *, steps: int, lead_passes: int = LEAD_PASSES,
    kernel_events: bool = False,
) -> list[LaunchStats]:
    """Per-launch device durations: an event pair for every launch of
    ``steps`` passes over ``calls`` (name, alg_bytes, thunk).

    By default the pair is recorded around the call (a marker packet on each
    side of the kernel). With ``kernel_events`` each thunk must make exactly
    one launch through the kernel library, and the pair is bound to that
    launch's own dispatch (``ako_time_next_launch``): the elapsed time is the
    kernel's start-to-end time, the duration a kernel trace records, and no
    marker packets sit between the kernels. A thunk that made no library
    launch raises.

    ``lead_passes`` untimed passes over the same calls are queued ahead of
    the timed ones without a wait, so the first timed launch follows the same
    kernels as every later one, on a device that has been busy all along:
    after the host-side pause before this region (event creation, the
    synchronisation), the first few passes ran up to 15% slower on MI355X
    while the device came back to its loaded clocks, which the 20-launch
    means of the largest cells then carried."""
    stream = torch.cuda.current_stream()
    marks = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in calls] for _ in range(steps)]
    if kernel_events:
        from ako_amd import _native

        # torch creates an event at its first record; record every one now,
        # outside the timed passes, so that each has a handle to arm.
        for pairs in marks:
            for ev0, ev1 in pairs:
                ev0.record(stream)
                ev1.record(stream)
    torch.cuda.synchronize()
    queue_lead()
    for _ in range(lead_passes):
        for _, _, fn in calls:
            fn()
    for step in range(steps):
        for (name, _, fn), (ev0, ev1) in zip(calls, marks[step]):
            if kernel_events:
                _native.time_next_launch(ev0, ev1)
                fn()
                if _native.disarm_launch_timing():
                    raise RuntimeError(f"time_each_launch: {name} made no launch through the kernel library")
            else:
                ev0.record(stream)
                fn()
                ev1.record(stream)
    torch.cuda.synchronize()
    stats: dict[str, LaunchStats] = {}
    for step in range(steps):
        for (name, nbytes, _), (ev0, ev1) in zip(calls, marks[step]):
            stats.setdefault(name, LaunchStats(name, nbytes)).durations_ms.append(ev0.elapsed_time(ev1))
    return list(stats.values())


def warm(calls: Sequence[tuple[str, int, Callable[[], Any]]], passes: int) -> None:
    for _ in range(passes):
        for _, _, fn in calls:
            fn()
    torch.cuda.synchronize()


def time_graph_replay(fn: Callable[[], Any], *, launches: int = 64, replays: int = 5) -> float:
    """Device microseconds per call with host overhead removed: ``launches``
    calls of ``fn`` are captured into one HIP graph, the graph is replayed
    ``replays`` times between two events, and the time is divided by the
    number of calls. Only kernels (no memsets) may be in ``fn``."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(launches):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    queue_lead()
    graph.replay()  # untimed, ahead of the first event: the timed replays follow the same work
    begin.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return begin.elapsed_time(end) * 1e3 / (launches * replays)


def time_back_to_back(fns: Sequence[Callable[[], Any]], *, launches: int) -> float:
    """Mean device milliseconds per call over ``launches`` back-to-back calls
    cycling through ``fns`` (independent input copies), one event pair around
    the whole loop: for kernels short enough that per-launch events would
    distort them. One untimed cycle through ``fns`` is queued ahead of the
    first event (after the spin lead), so the timed calls continue a cycle
    already running: every call still finds its inputs cold, and the device
    is at its loaded clocks from the first timed call on."""
    stream = torch.cuda.current_stream()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    queue_lead()
    for fn in fns:
        fn()
    begin.record(stream)
    for i in range(launches):
        fns[i % len(fns)]()
    end.record(stream)
    torch.cuda.synchronize()
    return begin.elapsed_time(end) / launches


def settled_back_to_back(fns: Sequence[Callable[[], Any]], *, launches: int, discard: int = 2,
                         keep: int = 3) -> float:
    """The median of ``keep`` ``time_back_to_back`` timings, after ``discard``
    more whose results are dropped. Right after a cell's inputs are
    allocated, the first 60-launch timings of MI355X read low and settle over
    the next two or three (residual RMSNorm 16384 x 8192: 79.7%, 80.5%, then
    80.7-80.8% of peak); the discarded runs cover that."""
    for _ in range(discard):
        time_back_to_back(fns, launches=launches)
    return statistics.median(time_back_to_back(fns, launches=launches) for _ in range(keep))


def parse_copy_ceiling(text: str) -> dict[str, Any] | None:
    """The fastest block shape among the JSON lines printed by ``copy_ceiling``
    for one size (None when there are none)."""
    import json

    rows = []
    for line in text.splitlines():
        line = line.strip()
        if line.startswith("{"):
            rows.append(json.loads(line))
    if not rows:
        return None
    best = dict(max(rows, key=lambda r: r["gbps"]))
    timed_b2b = [r for r in rows if "b2b_gbps" in r]
    if timed_b2b:
        b2b = max(timed_b2b, key=lambda r: r["b2b_gbps"])
        best["best_b2b_gbps"] = b2b["b2b_gbps"]
        best["best_b2b_frac"] = b2b["b2b_frac"]
    return best


def copy_same_bytes(alg_bytes: int, *, timeout_s: float = 120.0) -> dict[str, Any] | None:
    """Time a plain device copy that moves about ``alg_bytes`` (half read, half
    written) with ``ako_amd/_lib/copy_ceiling``, run as a child process.

    It is the reference for a streaming kernel of that size (what the plainest
    stream of those bytes reaches; a kernel that orders its traffic otherwise
    can pass it): launches pay a roughly fixed ramp-up, so the copy's share of
    the HBM peak falls with the byte count. Returns the probe's record for its fastest block shape, or
    None when the probe is not built or fails (it is a reference figure, not
    part of any result)."""
    import subprocess

    from ako_amd._build import COPY_PROBE_PATH

    per_buffer = (int(alg_bytes) // 2) // 16 * 16
    if per_buffer < 16 or not COPY_PROBE_PATH.exists():
        return None
    try:
        proc = subprocess.run([str(COPY_PROBE_PATH), str(per_buffer)], capture_output=True, text=True,
                              timeout=timeout_s)
    except (OSError, subprocess.TimeoutExpired):
        return None
    if proc.returncode != 0:
        return None
    return parse_copy_ceiling(proc.stdout)


def _capture(thunks: Sequence[Callable[[], Any]]) -> "torch.cuda.CUDAGraph":
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for fn in thunks:
                fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in thunks:
            fn()
    torch.cuda.synchronize()
    return graph


def _time_replays(graph: "torch.cuda.CUDAGraph", replays: int) -> float:
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    graph.replay()
    torch.cuda.synchronize()
    queue_lead()
    graph.replay()  # untimed, ahead of the first event: the timed replays follow the same work
    begin.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return begin.elapsed_time(end) / replays


def time_graph_cold(fns: Sequence[Callable[[], Any]], *, evict_bytes: int | None = None,
                    replays: int = 4, rounds: int = 5) -> float:
    """Device microseconds per call when every call finds its inputs in no cache.

    ``fns`` are calls on independent input copies (up to 64 are used). One HIP
    graph holds an eviction pass followed by one call of each; a second graph
    holds the eviction pass alone. The eviction is an elementwise
    read-modify-write (torch's ``add_``, a plain kernel: no memset is
    recorded) of a buffer of twice the L2s plus the Infinity Cache, so after
    it no input of the calls is cached anywhere. The cold cost per call is the
    difference of the two graphs' replay times over the number of calls: the
    median over ``rounds`` alternating measurements.
    """
    calls = list(fns)[:64]
    if evict_bytes is None:
        evict_bytes = 2 * CACHE_BYTES.get(device_arch() or "", CACHE_BYTES["gfx950"])
    scratch = torch.zeros(max(1, evict_bytes // 4), dtype=torch.float32, device=torch.cuda.current_device())

    def evict() -> None:
        scratch.add_(1.0)

    with_calls = _capture([evict, *calls])
    alone = _capture([evict])
    diffs = []
    for _ in range(rounds):
        t_both = _time_replays(with_calls, replays)
        t_evict = _time_replays(alone, replays)
        diffs.append((t_both - t_evict) * 1e3 / len(calls))
    del with_calls, alone, scratch
    return statistics.median(diffs)


def time_graph_after_producer(pairs: Sequence[tuple[Callable[[], Any], Callable[[], Any]]], *,
                              replays: int = 4, rounds: int = 5) -> float:
    """Device microseconds one call adds to a graph in which it runs the way a
    model runs it: right behind the kernel that writes its input.

    ``pairs`` are ``(producer, call)``: the producer (e.g. the projection GEMV
    whose output row the call normalises) writes the buffer the call reads,
    and every pair has buffers of its own, enough of them that one pass over
    the pairs streams far more than the caches hold. One HIP graph holds
    ``producer, call`` for every pair, a second the producers alone; the cost
    per call is the difference of their replay times over the number of
    pairs: the median over ``rounds`` alternating measurements. It includes
    what the call's launch costs behind a dependent kernel and its reads of
    a row another kernel has just written, which a graph of the call alone
    does not show."""
    pairs = list(pairs)
    both = _capture([fn for pair in pairs for fn in pair])
    alone = _capture([producer for producer, _ in pairs])
    diffs = []
    for _ in range(rounds):
        t_both = _time_replays(both, replays)
        t_alone = _time_replays(alone, replays)
        diffs.append((t_both - t_alone) * 1e3 / len(pairs))
    del both, alone
    return statistics.median(diffs)
