"""HIP candidate for ``swiglu`` (gfx950 kernel).

Drop-in replacement of ``swiglu_triton`` (``ako/ops/swiglu_triton.py:55-81``):
``fn(gate, up)`` returning a fresh tensor of gate's shape and dtype. No width
limit (the Triton wrapper raised above 65536).
"""

from __future__ import annotations

import torch

from ako_amd import _native
from ako_amd.ops._hip_common import call, dtype_code, empty_out, gpu_index, lib, raw_stream, rows_view


def swiglu_hip(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    fast = _native.torch_binding()
    if fast is not None:
        return fast.swiglu(gate, up)
    return swiglu_hip_ctypes(gate, up)


def swiglu_hip_ctypes(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``swiglu_hip`` with the host work in Python and the call through ctypes."""
    index = gpu_index(gate, "swiglu_hip")
    if gate.shape != up.shape:
        raise ValueError(f"Shape mismatch: gate {tuple(gate.shape)} vs up {tuple(up.shape)}")
    if up.dtype != gate.dtype or not up.is_cuda or up.get_device() != index:
        raise ValueError("swiglu_hip: up must match gate in dtype and device")
    dt = dtype_code(gate.dtype, "swiglu_hip")
    n = gate.shape[-1] if gate.dim() else 1
    gv, sg = rows_view(gate)
    uv, su = rows_view(up)
    rows = gv.numel() // n if n else 0
    y = empty_out(gate)
    status = call(index, lib().ako_swiglu_fwd, gv.data_ptr(), uv.data_ptr(), y.data_ptr(), rows, n,
                  sg, su, n, dt, raw_stream(index))
    if status:
        _native.check(status, "swiglu_hip")
    return y
