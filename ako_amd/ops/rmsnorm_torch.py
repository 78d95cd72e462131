"""Stronger PyTorch baselines: ``F.rms_norm`` and ``torch.compile`` of the references.

Same set and switches as ``ako/ops/rmsnorm_torch.py:37-78``,
``rope_torch.py:26-38`` and ``swiglu_torch.py:25-34``: the fused native
kernel is always a candidate when PyTorch has it (>= 2.4); the compiled
variants are opt-in through ``AKO_ENABLE_COMPILE=1`` because their first call
compiles for seconds. Beating these, not the unfused reference, is the claim.
"""

from __future__ import annotations

import os
from typing import Any, Callable

import torch
import torch.nn.functional as F

from ako_amd.ops.rmsnorm_ref import rmsnorm_ref, rmsnorm_residual_ref
from ako_amd.ops.rope_ref import rope_ref
from ako_amd.ops.swiglu_ref import swiglu_ref

_compiled: dict[str, Callable[..., Any]] = {}


def is_native_available() -> bool:
    return hasattr(F, "rms_norm")


def is_compile_enabled() -> bool:
    return os.environ.get("AKO_ENABLE_COMPILE", "").strip().lower() in {"1", "true", "yes", "on"}


def rmsnorm_torch_native(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    if not is_native_available():
        raise RuntimeError("torch.nn.functional.rms_norm requires PyTorch >= 2.4")
    return F.rms_norm(x, (x.shape[-1],), weight, eps)


def _compiled_fn(name: str, fn: Callable[..., Any]) -> Callable[..., Any]:
    if name not in _compiled:
        _compiled[name] = torch.compile(fn, dynamic=True)
    return _compiled[name]


def rmsnorm_compiled(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return _compiled_fn("rmsnorm", rmsnorm_ref)(x, weight, eps)


def rmsnorm_residual_compiled(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    return _compiled_fn("rmsnorm_residual", rmsnorm_residual_ref)(x, residual, weight, eps)


def rope_compiled(
    x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str = "neox"
) -> torch.Tensor:
    return _compiled_fn("rope", rope_ref)(x, cos, sin, style)


def swiglu_compiled(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return _compiled_fn("swiglu", swiglu_ref)(gate, up)


def reset_compiled_cache() -> None:
    _compiled.clear()
