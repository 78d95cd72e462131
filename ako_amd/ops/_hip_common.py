"""Shared host-side plumbing of the HIP candidates (tensor -> C-ABI arguments).

The candidates keep the reference's contract (``docs/EXTENDING.md:90-95`` of
Farx1/AKO): positional arguments, fresh outputs of the input's shape and
dtype, inputs never written, ``ValueError`` for bad arguments and
``RuntimeError`` for device failures. Work goes on torch's current stream of
the input's device, without synchronising.
"""

from __future__ import annotations

import contextlib
from typing import Iterator

import torch

from ako_amd import _native

_get_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)


def require_gpu(t: torch.Tensor, fn_name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{fn_name} requires a GPU tensor, got device {t.device}")


def dtype_code(dtype: torch.dtype, fn_name: str) -> int:
    code = _native.DTYPE_CODES.get(dtype)
    if code is None:
        raise ValueError(f"{fn_name} supports float32/float16/bfloat16, got {dtype}")
    return code


def raw_stream(device: torch.device) -> int:
    if _get_raw_stream is not None:
        return _get_raw_stream(device.index if device.index is not None else 0)
    return torch.cuda.current_stream(device).cuda_stream


@contextlib.contextmanager
def on_device(device: torch.device) -> Iterator[None]:
    """Make ``device`` current for the launch when it is not already."""
    current = _get_device() if _get_device is not None else torch.cuda.current_device()
    if device.index is None or device.index == current:
        yield
    else:
        with torch.cuda.device(device):
            yield


def rows_view(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """``(tensor, row_stride)`` such that row r of the last dimension starts at
    ``r * row_stride``; copies only when the leading dims cannot be walked with
    one stride or the last dimension is not contiguous."""
    if t.is_contiguous():
        return t, t.shape[-1] if t.dim() else 1
    if t.dim() >= 2 and t.stride(-1) == 1:
        row_stride = t.stride(-2)
        ok = True
        for i in range(t.dim() - 2):
            if t.shape[i] != 1 and t.stride(i) != t.stride(i + 1) * t.shape[i + 1]:
                ok = False
                break
        if ok and (t.shape[-2] == 1 or row_stride >= t.shape[-1]):
            return t, row_stride
    t = t.contiguous()
    return t, t.shape[-1]
