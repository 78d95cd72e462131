"""HIP candidates for ``rope`` (and a one-launch ``rope_qk``), gfx950 kernels.

``rope_hip(x, cos, sin, style)`` is the drop-in replacement of
``rope_triton`` (``ako/ops/rope_triton.py:97-156``). It accepts ``style``
positionally or as the ``style=`` keyword, as the selector passes it
(``ako/dispatcher/selector.py:285,293-300``). ``x`` may be any strided
``(batch, seq, heads, head_dim)`` view whose last dimension is contiguous
(e.g. ``q`` sliced out of a fused QKV projection): no copy is made. The
tables may be fp32, fp16 or bf16 regardless of x's dtype.

``rope_qk_hip`` rotates a query/key pair in a single launch; the reference's
``rope_qk`` issues two (``ako/ops/rope.py:45-58``). ``rope_qk_cache_hip`` also
writes the rotated keys and the values into a KV cache in that launch.
"""

from __future__ import annotations

import ctypes

import torch

from ako_amd import _native
from ako_amd.ops._hip_common import DT, call, dtype_code, gpu_index, lib, raw_stream
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
    fast = _native.torch_binding()
    if fast is not None:
        return fast.rope(x, cos, sin, style)
    return rope_hip_ctypes(x, cos, sin, style)


def rope_hip_ctypes(
    x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str = "neox"
) -> torch.Tensor:
    """``rope_hip`` with the host work in Python and the call through ctypes."""
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
    fast = _native.torch_binding()
    if fast is not None:
        return fast.rope_qk(q, k, cos, sin, style)
    return rope_qk_hip_ctypes(q, k, cos, sin, style)


def rope_qk_hip_ctypes(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str = "neox"
) -> tuple[torch.Tensor, torch.Tensor]:
    """``rope_qk_hip`` with the host work in Python and the call through ctypes."""
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


_I64x15 = ctypes.c_int64 * 15
# Stride arrays by stride tuples: a decoder calls this with the same few layouts
# every step. The arrays are read-only once built (the library copies the
# strides during the call), so sharing them between threads is safe.
_strides_cache: dict[tuple, ctypes.Array] = {}


def _cache_args_error(q, k, v, cos, sin, pos, k_cache, v_cache, style) -> str:
    """The first thing wrong with rope_qk_cache_hip's arguments (slow path)."""
    if style not in _native.ROPE_STYLE_CODES:
        return f"Unknown RoPE style {style!r}"
    if q.dim() != 4 or k.dim() != 4 or k_cache.dim() != 4:
        return "q, k and k_cache must be 4-D"
    batch, seq, _, head_dim = q.shape
    kv_heads = k.shape[2]
    if tuple(k.shape) != (batch, seq, kv_heads, head_dim) or k.dtype != q.dtype:
        return f"k {tuple(k.shape)} {k.dtype} does not match q {tuple(q.shape)} {q.dtype}"
    if (tuple(k_cache.shape) != (batch, kv_heads, k_cache.shape[2], head_dim)
            or k_cache.dtype != q.dtype):
        return (f"k_cache {tuple(k_cache.shape)} {k_cache.dtype} is not "
                f"(batch, kv_heads, cache_len, head_dim) of {q.dtype}")
    if (v is None) != (v_cache is None):
        return "v and v_cache must both be given or both be None"
    if v is not None and (tuple(v.shape) != tuple(k.shape) or v.dtype != q.dtype
                          or tuple(v_cache.shape) != tuple(k_cache.shape) or v_cache.dtype != q.dtype
                          or v_cache.stride() != k_cache.stride()):
        return "v / v_cache must match k / k_cache (shapes, dtype, strides)"
    if cos.dim() != 2 or cos.shape[1] != head_dim // 2 or sin.shape != cos.shape:
        return f"tables must be (positions, {head_dim // 2}), got {tuple(cos.shape)}"
    if pos.dtype != torch.int64 or pos.numel() < 1:
        return "pos must be an int64 tensor holding the position"
    index = q.get_device()
    for name, t in (("k", k), ("k_cache", k_cache), ("pos", pos)) + (
            (("v", v), ("v_cache", v_cache)) if v is not None else ()):
        if not t.is_cuda or t.get_device() != index:
            return f"{name} must be on the device of q"
    if k_cache.stride(-1) != 1 or (v_cache is not None and v_cache.stride(-1) != 1):
        return "cache rows must be contiguous in head_dim"
    return "unsupported arguments"


def rope_qk_cache_hip(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor | None,
    cos: torch.Tensor,
    sin: torch.Tensor,
    pos: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor | None,
    style: str = "neox",
) -> torch.Tensor:
    """One launch: rotated q out, rotated k and unrotated v into slot ``pos[0] + s``
    of the heads-major ``(batch, kv_heads, cache_len, head_dim)`` caches.

    ``pos`` stays on the device and is read by the kernel, so the launch can
    be captured in a HIP graph while the position advances between replays.
    Tokens whose slot falls outside the cache are not written (the host
    cannot see ``pos`` without a synchronisation); callers keep
    ``pos + seq <= cache_len``.
    """
    fast = _native.torch_binding()
    if fast is not None:
        return fast.rope_qk_cache(q, k, v, cos, sin, pos, k_cache, v_cache, style)
    return rope_qk_cache_hip_ctypes(q, k, v, cos, sin, pos, k_cache, v_cache, style)


def rope_qk_cache_hip_ctypes(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor | None,
    cos: torch.Tensor,
    sin: torch.Tensor,
    pos: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor | None,
    style: str = "neox",
) -> torch.Tensor:
    """``rope_qk_cache_hip`` with the host work in Python and the call through
    ctypes. The common case is checked with one combined test and the detailed
    message is only built when it fails."""
    index = gpu_index(q, "rope_qk_cache_hip")
    style_code = _native.ROPE_STYLE_CODES.get(style)
    qshape, kshape, cshape = q.shape, k.shape, k_cache.shape
    dt = DT.get(q.dtype)
    ok = (
        style_code is not None and dt is not None and len(qshape) == 4 and len(kshape) == 4
        and len(cshape) == 4 and kshape[0] == qshape[0] and kshape[1] == qshape[1]
        and kshape[3] == qshape[3] and cshape[0] == qshape[0] and cshape[1] == kshape[2]
        and cshape[3] == qshape[3] and k.dtype is q.dtype and k_cache.dtype is q.dtype
        and cos.dim() == 2 and cos.shape[1] * 2 == qshape[3] and sin.shape == cos.shape
        and pos.dtype is torch.int64 and pos.numel() >= 1 and k.is_cuda and k_cache.is_cuda and pos.is_cuda
        and k_cache.stride(3) == 1
    )
    if ok and v is not None:
        ok = (v_cache is not None and v.shape == kshape and v.dtype is q.dtype and v.is_cuda
              and v_cache.shape == cshape and v_cache.dtype is q.dtype and v_cache.is_cuda
              and v_cache.stride() == k_cache.stride())
    elif ok:
        ok = v_cache is None
    if not ok or k.get_device() != index or k_cache.get_device() != index or pos.get_device() != index:
        raise ValueError("rope_qk_cache_hip: " + _cache_args_error(q, k, v, cos, sin, pos, k_cache, v_cache, style))
    batch, seq, q_heads, head_dim = qshape
    qv, kv = _head_view(q), _head_view(k)
    vv = _head_view(v) if v is not None else None
    tdt = cos.dtype
    if tdt is sin.dtype and tdt in DT and cos.is_contiguous() and sin.is_contiguous() \
            and cos.is_cuda and cos.get_device() == index and sin.get_device() == index:
        c, s, st = cos, sin, cos.shape[1]  # the common case: one dense table pair
    else:
        c, s, st = _table_stride(_table(cos, index), _table(sin, index))
    q_out = torch.empty_like(q) if q.is_contiguous() else torch.empty(qshape, dtype=q.dtype, device=q.device)
    key = (qv.stride(), kv.stride(), vv.stride() if vv is not None else None, q_out.stride(),
           k_cache.stride())
    strides = _strides_cache.get(key)
    if strides is None:
        qs, ks, vs, qos, cs = key
        vs = vs or (0, 0, 0, 0)
        strides = _I64x15(qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
                          qos[0], qos[1], qos[2], cs[0], cs[2], cs[1])
        if len(_strides_cache) < 256:
            _strides_cache[key] = strides
    base = _addressof(strides)
    status = call(
        index, lib().ako_rope_qk_cache_fwd,
        qv.data_ptr(), kv.data_ptr(), vv.data_ptr() if vv is not None else None,
        c.data_ptr(), s.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr() if v_cache is not None else None, pos.data_ptr(),
        batch, seq, q_heads, kshape[2], head_dim,
        base, base + 24, base + 48, base + 72, base + 96,
        cshape[2], c.shape[0], st, dt, _native.DTYPE_CODES[c.dtype], style_code,
        raw_stream(index),
    )
    if status:
        _native.check(status, "rope_qk_cache_hip")
    return q_out
