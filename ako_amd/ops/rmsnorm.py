"""Public RMSNorm operations with adaptive kernel selection.

Signatures and dispatch follow ``ako/ops/rmsnorm.py:11-56``.
"""

from __future__ import annotations

import torch

from ako_amd.dispatcher.selector import get_selector
from ako_amd.ops._registry import register_all


def rmsnorm(
    x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, *, kernel: str | None = None
) -> torch.Tensor:
    """RMSNorm over the last dimension; ``kernel`` forces an implementation by name."""
    register_all()
    fn = get_selector().select("rmsnorm", x, weight, forced=kernel)
    return fn(x, weight, eps)


def rmsnorm_residual(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    *,
    kernel: str | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(rmsnorm(x + residual), x + residual)``."""
    register_all()
    fn = get_selector().select("rmsnorm_residual", x, residual, weight, forced=kernel)
    return fn(x, residual, weight, eps)
