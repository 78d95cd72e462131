"""HIP candidates for ``rope`` (and a one-launch ``rope_qk``), gfx950 kernels.

``rope_hip(x, cos, sin, style)`` is the drop-in replacement of
``rope_triton`` (``ako/ops/rope_triton.py:97-156``). It accepts ``style``
positionally or as the ``style=`` keyword, as the selector passes it
(``ako/dispatcher/selector.py:285,293-300``). ``x`` may be any strided
``(batch, seq, heads, head_dim)`` view whose last dimension is contiguous
(e.g. ``q`` sliced out of a fused QKV projection): no copy is made. The
tables may be fp32, fp16 or bf16 regardless of x's dtype.

``rope_qk_hip`` rotates a query/key pair in a single launch; the reference's
``rope_qk`` issues two (``ako/ops/rope.py:45-58``).
"""

from __future__ import annotations

import ctypes

import torch

from ako_amd import _native
from ako_amd.ops._hip_common import call, dtype_code, gpu_index, lib, raw_stream
from ako_amd.ops.rope_ref import validate_rope_args


def _head_view(x: torch.Tensor) -> torch.Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


def _table(t: torch.Tensor, index: int) -> torch.Tensor:
    if not t.is_cuda or t.get_device() != index:
        raise ValueError(f"rope_hip: tables must be on the input's device, got {t.device}")
    if t.dtype not in _native.DTYPE_CODES:
        t = t.float()
    return t if t.stride(-1) == 1 else t.contiguous()


def _table_stride(cos: torch.Tensor, sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, int]:
    # One row stride serves both tables; make them agree when they do not.
    if cos.stride(0) != sin.stride(0) or cos.dtype != sin.dtype:
        cos, sin = cos.contiguous(), sin.to(cos.dtype).contiguous()
    return cos, sin, cos.stride(0) if cos.shape[0] > 1 else cos.shape[1]


def rope_hip(
    x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str = "neox"
) -> torch.Tensor:
    index = gpu_index(x, "rope_hip")
    validate_rope_args(x, cos, sin, style)
    dt = dtype_code(x.dtype, "rope_hip")
    xv = _head_view(x)
    c, s, st = _table_stride(_table(cos, index), _table(sin, index))
    batch, seq, heads, head_dim = x.shape
    y = torch.empty_like(x) if x.is_contiguous() else torch.empty(x.shape, dtype=x.dtype, device=x.device)
    status = call(
        index, lib().ako_rope_fwd,
        xv.data_ptr(), c.data_ptr(), s.data_ptr(), y.data_ptr(),
        batch, seq, heads, head_dim,
        xv.stride(0), xv.stride(1), xv.stride(2),
        y.stride(0), y.stride(1), y.stride(2),
        st, dt, _native.DTYPE_CODES[c.dtype], _native.ROPE_STYLE_CODES[style],
        raw_stream(index),
    )
    if status:
        _native.check(status, "rope_hip")
    return y


_addressof = ctypes.addressof
_I64x12 = ctypes.c_int64 * 12


def rope_qk_hip(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str = "neox"
) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate ``q`` and ``k`` (same batch, seq, head_dim and dtype) in one launch."""
    index = gpu_index(q, "rope_qk_hip")
    validate_rope_args(q, cos, sin, style)
    validate_rope_args(k, cos, sin, style)
    if (q.shape[:2] != k.shape[:2] or q.shape[3] != k.shape[3] or q.dtype != k.dtype
            or not k.is_cuda or k.get_device() != index):
        raise ValueError(
            f"rope_qk_hip: q {tuple(q.shape)} {q.dtype} and k {tuple(k.shape)} {k.dtype} differ"
        )
    dt = dtype_code(q.dtype, "rope_qk_hip")
    qv, kv = _head_view(q), _head_view(k)
    c, s, st = _table_stride(_table(cos, index), _table(sin, index))
    batch, seq, q_heads, head_dim = q.shape
    q_out = torch.empty_like(q) if q.is_contiguous() else torch.empty(q.shape, dtype=q.dtype, device=q.device)
    k_out = torch.empty_like(k) if k.is_contiguous() else torch.empty(k.shape, dtype=k.dtype, device=k.device)
    qs, ks, qos, kos = qv.stride(), kv.stride(), q_out.stride(), k_out.stride()
    strides = _I64x12(qs[0], qs[1], qs[2], ks[0], ks[1], ks[2],
                      qos[0], qos[1], qos[2], kos[0], kos[1], kos[2])
    base = _addressof(strides)
    status = call(
        index, lib().ako_rope_qk_fwd,
        qv.data_ptr(), kv.data_ptr(), c.data_ptr(), s.data_ptr(),
        q_out.data_ptr(), k_out.data_ptr(), batch, seq, q_heads, k.shape[2], head_dim,
        base, base + 24, base + 48, base + 72,
        st, dt, _native.DTYPE_CODES[c.dtype], _native.ROPE_STYLE_CODES[style],
        raw_stream(index),
    )
    if status:
        _native.check(status, "rope_qk_hip")
    return q_out, k_out
