"""GPU: the launch-timing hook (ako_time_next_launch).

An armed event pair is taken by exactly the next launch the thread makes
through the library, and that launch's results are those of an unarmed call.
The pair's elapsed time lies inside an event pair recorded around the call.
A later unarmed launch leaves the pair alone, and a thunk that makes no
library launch is refused by the per-launch timer.
"""

from __future__ import annotations

import pytest
import torch

from ako_amd import _native
from ako_amd.benchmark import roofline as rf
from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
from ako_amd.ops.rope_hip import rope_qk_hip
from ako_amd.ops.rope_ref import build_rope_tables
from ako_amd.ops.swiglu_hip import swiglu_hip

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]
DEV = "cuda"


def _rand(*shape, dtype=torch.float16, seed=0, scale=1.0, shift=0.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV) * scale + shift).to(dtype)


def _cases():
    x = _rand(4096, 4096)
    r = _rand(4096, 4096, seed=1)
    w = _rand(4096, seed=2, scale=0.1, shift=1.0)
    q = _rand(2, 512, 32, 128, dtype=torch.bfloat16, seed=3)
    k = _rand(2, 512, 8, 128, dtype=torch.bfloat16, seed=4)
    cos, sin = build_rope_tables(512, 128, device=DEV)
    g = _rand(1024, 4096, dtype=torch.bfloat16, seed=5)
    u = _rand(1024, 4096, dtype=torch.bfloat16, seed=6)
    return {
        "rmsnorm": lambda: rmsnorm_hip(x, w),
        "rmsnorm_residual": lambda: rmsnorm_residual_hip(x, r, w),
        "rope_qk": lambda: rope_qk_hip(q, k, cos, sin),
        "swiglu": lambda: swiglu_hip(g, u),
    }


def _flat(out):
    return list(out) if isinstance(out, tuple) else [out]


def _recorded_pair():
    pair = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for ev in pair:
        ev.record()
    torch.cuda.synchronize()
    return pair


@pytest.mark.parametrize("op", ["rmsnorm", "rmsnorm_residual", "rope_qk", "swiglu"])
def test_armed_pair_times_exactly_the_next_launch(op) -> None:
    fn = _cases()[op]
    want = _flat(fn())
    start, stop = _recorded_pair()
    outer0, outer1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    outer0.record()
    _native.time_next_launch(start, stop)
    got = _flat(fn())
    outer1.record()
    assert not _native.disarm_launch_timing(), "the launch did not take the armed pair"
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    kernel_ms = start.elapsed_time(stop)
    around_ms = outer0.elapsed_time(outer1)
    assert 0.0 < kernel_ms <= around_ms, (kernel_ms, around_ms)
    fn()  # unarmed: the pair keeps the first launch's times
    torch.cuda.synchronize()
    assert start.elapsed_time(stop) == kernel_ms


def test_kernel_events_refuse_a_thunk_without_a_library_launch() -> None:
    x = torch.zeros(1024, device=DEV)
    with pytest.raises(RuntimeError, match="no launch through the kernel library"):
        rf.time_each_launch([("fill", 4096, lambda: x.add_(1.0))], steps=1, lead_passes=0, kernel_events=True)
    assert not _native.disarm_launch_timing()


def test_kernel_events_per_launch_means() -> None:
    """time_each_launch with kernel-bound events against marker events on the
    same calls: every launch recorded, each kernel-bound mean positive and no
    larger than the marker-bracketed mean plus 1% (the two runs are separate
    passes, so a launch may run a little slower in the second)."""
    cases = _cases()
    calls = [(name, 1, fn) for name, fn in cases.items()]
    marker = {s.name: s for s in rf.time_each_launch(calls, steps=5)}
    bound = {s.name: s for s in rf.time_each_launch(calls, steps=5, kernel_events=True)}
    for name in cases:
        assert len(bound[name].durations_ms) == 5
        assert 0.0 < bound[name].mean_ms <= marker[name].mean_ms * 1.01, (name, bound[name].mean_ms,
                                                                          marker[name].mean_ms)
