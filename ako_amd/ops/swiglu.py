"""Public SwiGLU operation with adaptive kernel selection (``ako/ops/swiglu.py:11-24``)."""

from __future__ import annotations

import torch

from ako_amd.dispatcher.selector import get_selector
from ako_amd.ops._registry import register_all


def swiglu(gate: torch.Tensor, up: torch.Tensor, *, kernel: str | None = None) -> torch.Tensor:
    """``silu(gate) * up``."""
    register_all()
    fn = get_selector().select("swiglu", gate, up, forced=kernel)
    return fn(gate, up)


__all__ = ["swiglu"]
