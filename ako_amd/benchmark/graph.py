"""HIP-graph capture of one kernel call (decode-sized rows).

Same contract as ``ako/benchmark/graph.py:31-67``: warm up on a side stream
with the caller's tensors alive, capture one call, and hand back a replay
callable; any failure (an op that allocates unpredictably, no device) is
returned as an uncaptured result with a reason instead of raising. Under
PyTorch-ROCm ``torch.cuda.CUDAGraph`` records a hipGraph.

The side stream is created at default priority (the only priority used
anywhere in this package).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch


@dataclass
class CapturedKernel:
    replay: Callable[[], None] | None
    captured: bool
    reason: str | None = None
    graph: Any = None


def try_capture(
    fn: Callable[..., Any],
    args: tuple[Any, ...],
    kwargs: dict[str, Any] | None = None,
    *,
    warmup: int = 3,
) -> CapturedKernel:
    """Capture ``fn(*args, **kwargs)`` into a graph if the device allows it."""
    kwargs = kwargs or {}
    x = args[0] if args else None
    if not isinstance(x, torch.Tensor) or not x.is_cuda:
        return CapturedKernel(None, False, "not_cuda")
    if not hasattr(torch.cuda, "CUDAGraph"):
        return CapturedKernel(None, False, "graph_unavailable")
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                fn(*args, **kwargs)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn(*args, **kwargs)
        torch.cuda.synchronize()
    except RuntimeError as exc:
        return CapturedKernel(None, False, f"{type(exc).__name__}: {exc}")
    return CapturedKernel(graph.replay, True, graph=graph)
