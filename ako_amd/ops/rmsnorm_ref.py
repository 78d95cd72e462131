"""Unfused PyTorch RMSNorm: the specification and the gate's reference.

Restates ``ako/ops/rmsnorm_ref.py:8-50``. Half-precision inputs are upcast to
fp32, every intermediate is materialised (so this is ~6-8 eager kernels), and
the result is cast back to the input dtype:

    y = ((x * rsqrt(mean(x**2, -1) + eps)) * w).to(x.dtype)

The residual variant adds in the *storage* dtype first (``x + residual`` in
fp16 rounds the sum to fp16) and normalises that rounded sum.
"""

from __future__ import annotations

import torch

_HALF = (torch.float16, torch.bfloat16)


def rmsnorm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    compute = torch.float32 if x.dtype in _HALF else x.dtype
    xc = x.to(compute)
    variance = xc.pow(2).mean(dim=-1, keepdim=True)
    normed = xc * torch.rsqrt(variance + eps)
    return (normed * weight.to(compute)).to(x.dtype)


def rmsnorm_residual_ref(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(rmsnorm(x + residual), x + residual)`` with the sum in the storage dtype."""
    if x.shape != residual.shape:
        raise ValueError(f"Shape mismatch: x {tuple(x.shape)} vs residual {tuple(residual.shape)}")
    new_residual = x + residual
    return rmsnorm_ref(new_residual, weight, eps), new_residual
