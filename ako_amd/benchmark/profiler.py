"""``torch.profiler`` wrapper (reference ``ako/benchmark/profiler.py:11-26``).

Kernel-level counters come from ``rocprofv3`` instead (``ako_amd.benchmark.rocprof``).
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any, Iterator

import torch


@contextmanager
def profile_cuda(activities: list[Any] | None = None) -> Iterator[torch.profiler.profile]:
    if activities is None:
        activities = [torch.profiler.ProfilerActivity.CPU]
        if torch.cuda.is_available():
            activities.append(torch.profiler.ProfilerActivity.CUDA)
    with torch.profiler.profile(activities=activities, record_shapes=True) as prof:
        yield prof
