"""Unfused PyTorch SwiGLU activation ``silu(gate) * up``.

Restates ``ako/ops/swiglu_ref.py:16-32``: half-precision inputs are upcast to
fp32, ``F.silu`` materialises an intermediate that the multiply reads back,
and the product is cast to the input dtype.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def swiglu_ref(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    if gate.shape != up.shape:
        raise ValueError(f"Shape mismatch: gate {tuple(gate.shape)} vs up {tuple(up.shape)}")
    compute = torch.float32 if gate.dtype in (torch.float16, torch.bfloat16) else gate.dtype
    return (F.silu(gate.to(compute)) * up.to(compute)).to(gate.dtype)
