"""Helpers shared by the tests: torch <-> oracle storage arrays, seeded inputs."""

from __future__ import annotations

import numpy as np
import torch

NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def to_np(t: torch.Tensor) -> np.ndarray:
    """A tensor in the oracle's storage format (bf16 as uint16 bit patterns)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def from_np(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.bfloat16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype)


def randn(shape, dtype: torch.dtype, seed: int, *, scale: float = 1.0, shift: float = 0.0,
          device: str = "cpu") -> torch.Tensor:
    """Seeded N(shift, scale^2) drawn in fp32 on the CPU, cast, then moved."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g) * scale + shift
    return t.to(dtype).to(device)
