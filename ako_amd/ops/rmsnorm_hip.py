"""HIP candidates for ``rmsnorm`` and ``rmsnorm_residual`` (gfx950 kernels).

Drop-in replacements of ``rmsnorm_triton`` / ``rmsnorm_residual_triton``
(``ako/ops/rmsnorm_triton.py:139-192``): same positional signatures, fresh
outputs, ``ValueError`` on bad input. Differences from the Triton wrappers:
no hidden-size limit, no copy of inputs whose rows are already strided
uniformly, and the weight may be fp32 for half-precision inputs (any other
weight dtype is widened to fp32, which is exact and what the reference's
``weight.to(float32)`` does).
"""

from __future__ import annotations

import torch

from ako_amd import _native
from ako_amd.ops._hip_common import (
    DT, call, dtype_code, empty_out, gpu_index, lib, raw_stream, rows_view,
)


def _weight(weight: torch.Tensor, index: int, dt: int, hidden: int, fn_name: str) -> tuple[torch.Tensor, int]:
    if weight.shape != (hidden,):
        raise ValueError(f"Expected weight of shape ({hidden},), got {tuple(weight.shape)}")
    if not weight.is_cuda or weight.get_device() != index:
        raise ValueError(f"{fn_name}: weight must be on the input's device")
    wdt = DT.get(weight.dtype)
    if wdt != dt and wdt != 0:  # neither the input dtype nor fp32
        weight, wdt = weight.float(), 0
    if not weight.is_contiguous():
        weight = weight.contiguous()
    return weight, wdt


def rmsnorm_hip(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last dimension on the GPU."""
    fast = _native.torch_binding()
    if fast is not None:
        return fast.rmsnorm(x, weight, eps)
    return rmsnorm_hip_ctypes(x, weight, eps)


def rmsnorm_hip_ctypes(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``rmsnorm_hip`` with the host work in Python and the call through ctypes."""
    index = gpu_index(x, "rmsnorm_hip")
    dt = dtype_code(x.dtype, "rmsnorm_hip")
    hidden = x.shape[-1] if x.dim() else 1
    w, wdt = _weight(weight, index, dt, hidden, "rmsnorm_hip")
    xv, sx = rows_view(x)
    rows = xv.numel() // hidden if hidden else 0
    y = empty_out(x)
    status = call(index, lib().ako_rmsnorm_fwd, xv.data_ptr(), w.data_ptr(), y.data_ptr(), rows,
                  hidden, sx, hidden, eps, dt, wdt, raw_stream(index))
    if status:
        _native.check(status, "rmsnorm_hip")
    return y


def rmsnorm_residual_hip(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(rmsnorm(x + residual), x + residual)`` with the sum rounded to x's dtype."""
    fast = _native.torch_binding()
    if fast is not None:
        return fast.rmsnorm_residual(x, residual, weight, eps)
    return rmsnorm_residual_hip_ctypes(x, residual, weight, eps)


def rmsnorm_residual_hip_ctypes(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """``rmsnorm_residual_hip`` with the host work in Python and the call through ctypes."""
    index = gpu_index(x, "rmsnorm_residual_hip")
    if x.shape != residual.shape:
        raise ValueError(f"Shape mismatch: x {tuple(x.shape)} vs residual {tuple(residual.shape)}")
    if residual.dtype != x.dtype or not residual.is_cuda or residual.get_device() != index:
        raise ValueError("rmsnorm_residual_hip: residual must match x in dtype and device")
    dt = dtype_code(x.dtype, "rmsnorm_residual_hip")
    hidden = x.shape[-1] if x.dim() else 1
    w, wdt = _weight(weight, index, dt, hidden, "rmsnorm_residual_hip")
    xv, sx = rows_view(x)
    rv, sr = rows_view(residual)
    rows = xv.numel() // hidden if hidden else 0
    y = empty_out(x)
    new_residual = empty_out(x)
    status = call(index, lib().ako_rmsnorm_residual_fwd, xv.data_ptr(), rv.data_ptr(), w.data_ptr(),
                  y.data_ptr(), new_residual.data_ptr(), rows, hidden, sx, sr, hidden, hidden,
                  eps, dt, wdt, raw_stream(index))
    if status:
        _native.check(status, "rmsnorm_residual_hip")
    return y, new_residual
