"""Shared host-side plumbing of the HIP candidates (tensor -> C-ABI arguments).

The candidates keep the reference's contract (``docs/EXTENDING.md:90-95`` of
Farx1/AKO): positional arguments, fresh outputs of the input's shape and
dtype, inputs never written, ``ValueError`` for bad arguments and
``RuntimeError`` for device failures. Work goes on torch's current stream of
the input's device, without synchronising.

The per-call host path is kept short because at decode sizes (one token) the
selector's wall-clock race against PyTorch eager is decided by host cost,
not by the kernel: no context managers, ``empty_like`` for contiguous
inputs, one ctypes call.
"""

from __future__ import annotations

import torch

from ako_amd import _native

DT = _native.DTYPE_CODES
_get_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)


def lib():
    """The loaded C-ABI library (raises ``HipLibraryError`` if unusable)."""
    return _native._lib or _native.load()


def gpu_index(t: torch.Tensor, fn_name: str) -> int:
    """Device index of a GPU tensor; ``ValueError`` for anything else."""
    if not t.is_cuda:
        raise ValueError(f"{fn_name} requires a GPU tensor, got device {t.device}")
    return t.get_device()


def dtype_code(dtype: torch.dtype, fn_name: str) -> int:
    code = DT.get(dtype)
    if code is None:
        raise ValueError(f"{fn_name} supports float32/float16/bfloat16, got {dtype}")
    return code


def raw_stream(index: int) -> int:
    """Raw ``hipStream_t`` of torch's current stream on device ``index``."""
    if _get_raw_stream is not None:
        return _get_raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def current_device() -> int:
    return _get_device() if _get_device is not None else torch.cuda.current_device()


def call(index: int, fn, *args) -> int:
    """Invoke a C-ABI entry with ``index`` as the current device."""
    if index == current_device():
        return fn(*args)
    with torch.cuda.device(index):
        return fn(*args)


def leading_row_stride(shape, strides) -> int | None:
    """Stride between consecutive rows of the last dimension when the leading
    dims (all but the last) can be walked as one run of equally spaced rows,
    else ``None``.

    Size-1 dims are transparent: their stride is arbitrary in torch and never
    multiplies an index. The innermost leading dim of size > 1 fixes the row
    stride; every outer one of size > 1 must then be that stride times the
    number of rows the dims inside it span. With at most one row the stride
    is the row length (it is never used to step)."""
    h = shape[-1] if len(shape) else 1
    row_stride = None
    spanned = 1
    for size, stride in zip(reversed(shape[:-1]), reversed(strides[:-1])):
        if size == 1:
            continue
        if row_stride is None:
            row_stride, spanned = stride, size
        elif stride != row_stride * spanned:
            return None
        else:
            spanned *= size
    if row_stride is None:
        return h
    return row_stride if row_stride >= h else None


def rows_view(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """``(tensor, row_stride)`` such that row r of the last dimension starts at
    ``r * row_stride``; copies only when the leading dims cannot be walked with
    one stride or the last dimension is not contiguous."""
    if t.is_contiguous():
        return t, t.shape[-1] if t.dim() else 1
    if t.dim() >= 2 and (t.stride(-1) == 1 or t.shape[-1] <= 1):
        row_stride = leading_row_stride(t.shape, t.stride())
        if row_stride is not None:
            return t, row_stride
    t = t.contiguous()
    return t, t.shape[-1]


def empty_out(x: torch.Tensor) -> torch.Tensor:
    """A fresh contiguous tensor of x's shape, dtype and device."""
    if x.is_contiguous():
        return torch.empty_like(x)
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)
