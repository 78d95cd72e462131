"""Replaying a run of kernel calls from one HIP graph.

At decode sizes a candidate's device time is a microsecond or two, well below
the host's launch cost, so a wall clock around eager launches measures the
launch path. ``capture_calls`` records one call per argument tuple into a
single ``torch.cuda.CUDAGraph`` (a hipGraph under PyTorch-ROCm); replaying it
issues all of them with one host call. Given several tuples (a rotation ring of
input copies) the replay also reads a different copy per call.

Capture follows PyTorch's documented recipe: the calls are first run on a side
stream, so that lazy initialisation and allocator growth happen outside the
capture, and the side stream joins the current one before capture starts. The
side stream keeps the default priority. A capture that fails (an operation that
synchronises or allocates in a way the graph cannot record, or no GPU) is not
an error: the result carries ``graph=None`` and the reason, and the caller
times eager launches instead. Used by the reference's measurement in the same
way (``ako/benchmark/graph.py:31-67``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable, Sequence

import torch


@dataclass
class GraphedCalls:
    """The outcome of a capture: ``replay()`` runs every recorded call once."""

    graph: Any
    calls: int
    reason: str | None = None

    def replay(self) -> None:
        if self.graph is None:
            raise RuntimeError(f"nothing was captured: {self.reason}")
        self.graph.replay()


def capture_calls(
    fn: Callable[..., Any],
    arg_sets: Sequence[tuple[Any, ...]],
    kwargs: dict[str, Any] | None = None,
    *,
    warmup: int = 2,
) -> GraphedCalls:
    """Record ``fn(*args, **kwargs)`` for each tuple of ``arg_sets`` into one graph."""
    kwargs = kwargs or {}
    if not arg_sets:
        return GraphedCalls(None, 0, "no calls to capture")
    first = arg_sets[0][0] if arg_sets[0] else None
    if not (isinstance(first, torch.Tensor) and first.is_cuda):
        return GraphedCalls(None, 0, "inputs are not on a GPU")
    side = torch.cuda.Stream(device=first.device)
    try:
        side.wait_stream(torch.cuda.current_stream(first.device))
        with torch.cuda.stream(side):
            for _ in range(max(1, warmup)):
                for args in arg_sets:
                    fn(*args, **kwargs)
        torch.cuda.current_stream(first.device).wait_stream(side)
        torch.cuda.synchronize(first.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for args in arg_sets:
                fn(*args, **kwargs)
        torch.cuda.synchronize(first.device)
    except RuntimeError as exc:
        torch.cuda.synchronize(first.device)
        return GraphedCalls(None, 0, f"{type(exc).__name__}: {exc}")
    return GraphedCalls(graph, len(arg_sets))
