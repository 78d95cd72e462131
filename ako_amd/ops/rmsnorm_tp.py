"""RMSNorm over a hidden dimension split across tensor-parallel ranks.

The reference normalises whole rows (``ako/ops/rmsnorm_ref.py:8-50``). Under
tensor parallelism each rank holds a slice of every row, and the mean of
squares needs every slice. The rank-local work splits in two:

1. ``rmsnorm_shard_partial``: ``s = x (+ residual)`` (rounded to the storage
   dtype, as the reference adds) and the fp32 sum of ``s**2`` over the slice,
   one float per row;
2. the per-row partial sums are summed over the ranks (one all-reduce of
   ``rows`` floats, 64 KiB for 16384 rows);
3. ``rmsnorm_shard_apply``: ``y = (s * rsqrt(total / hidden + eps)) * w`` on
   the slice, with ``hidden`` the full row length.

``rmsnorm_tp`` is one rank's part in a ``torch.distributed`` group: partial,
all-reduce, apply. ``rmsnorm_sharded`` runs every slice of a row on one
device and sums the partials with ``torch.sum`` where the ranks would
all-reduce them. That shows the
per-rank kernels at their real shapes and that the slices compose to the
full-row result. The HIP halves are ``ako_rmsnorm_shard_partial_fwd`` and
``ako_rmsnorm_shard_apply_fwd``; the ``*_ref`` functions are the same
arithmetic in PyTorch.
"""

from __future__ import annotations

from typing import Callable

import torch

from ako_amd import _native
from ako_amd.ops._hip_common import DT, call, dtype_code, empty_out, gpu_index, lib, raw_stream, rows_view


def _rows(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1] if x.shape[-1] else 0


def rmsnorm_shard_partial_ref(
    x: torch.Tensor, residual: torch.Tensor | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    s = x if residual is None else x + residual
    return s, s.float().pow(2).sum(-1)


def rmsnorm_shard_apply_ref(
    s: torch.Tensor, weight: torch.Tensor, total_ss: torch.Tensor, hidden: int, eps: float = 1e-6
) -> torch.Tensor:
    rstd = torch.rsqrt(total_ss * (1.0 / hidden) + eps)
    return ((s.float() * rstd.unsqueeze(-1)) * weight.float()).to(s.dtype)


def rmsnorm_shard_partial_hip(
    x: torch.Tensor, residual: torch.Tensor | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(s, partial_ss)`` for this rank's slice; ``s`` is ``x`` itself without a residual."""
    index = gpu_index(x, "rmsnorm_shard_partial_hip")
    dt = dtype_code(x.dtype, "rmsnorm_shard_partial_hip")
    shard = x.shape[-1]
    xv, sx = rows_view(x)
    rows = _rows(x)
    partial = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    if residual is None:
        s, rv, sr, rout, so = x, None, 0, None, 0
    else:
        if residual.shape != x.shape or residual.dtype != x.dtype or residual.device != x.device:
            raise ValueError("rmsnorm_shard_partial_hip: residual must match x in shape, dtype and device")
        rv, sr = rows_view(residual)
        s = empty_out(x)
        rout, so = s, shard
    status = call(index, lib().ako_rmsnorm_shard_partial_fwd, xv.data_ptr(),
                  rv.data_ptr() if rv is not None else None, rout.data_ptr() if rout is not None else None,
                  partial.data_ptr(), rows, shard, sx, sr, so, dt, raw_stream(index))
    if status:
        _native.check(status, "rmsnorm_shard_partial_hip")
    return s, partial


def rmsnorm_shard_apply_hip(
    s: torch.Tensor, weight: torch.Tensor, total_ss: torch.Tensor, hidden: int, eps: float = 1e-6
) -> torch.Tensor:
    """``y`` on this rank's slice, given the per-row sums of squares over the whole row."""
    index = gpu_index(s, "rmsnorm_shard_apply_hip")
    dt = dtype_code(s.dtype, "rmsnorm_shard_apply_hip")
    shard = s.shape[-1]
    if weight.shape != (shard,) or not weight.is_cuda or weight.get_device() != index:
        raise ValueError(f"rmsnorm_shard_apply_hip: weight must be ({shard},) on the input's device")
    wdt = DT.get(weight.dtype)
    if wdt != dt and wdt != 0:
        weight, wdt = weight.float(), 0
    weight = weight.contiguous()
    if total_ss.dtype != torch.float32 or total_ss.shape != s.shape[:-1] or total_ss.device != s.device:
        raise ValueError("rmsnorm_shard_apply_hip: total_ss must be float32 with one value per row")
    total_ss = total_ss.contiguous()
    sv, ssr = rows_view(s)
    y = empty_out(s)
    status = call(index, lib().ako_rmsnorm_shard_apply_fwd, sv.data_ptr(), weight.data_ptr(),
                  total_ss.data_ptr(), y.data_ptr(), _rows(s), shard, hidden, ssr, shard, eps, dt, wdt,
                  raw_stream(index))
    if status:
        _native.check(status, "rmsnorm_shard_apply_hip")
    return y


def rmsnorm_sharded(
    x: torch.Tensor,
    residual: torch.Tensor | None,
    weight: torch.Tensor,
    eps: float = 1e-6,
    *,
    shards: int,
    partial_fn: Callable = rmsnorm_shard_partial_hip,
    apply_fn: Callable = rmsnorm_shard_apply_hip,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Every rank's slice of ``(rmsnorm(x + residual), x + residual)`` on one device.

    The hidden dimension is cut into ``shards`` equal slices (the column
    layout of a tensor-parallel rank); ``torch.sum`` over the slices' partial
    sums stands in for the all-reduce. Returns the concatenated outputs.
    """
    hidden = x.shape[-1]
    if hidden % shards:
        raise ValueError(f"hidden {hidden} is not divisible by {shards} shards")
    width = hidden // shards
    cols = [slice(i * width, (i + 1) * width) for i in range(shards)]
    parts = [partial_fn(x[..., c], None if residual is None else residual[..., c]) for c in cols]
    total = torch.stack([p for _, p in parts]).sum(0)
    ys = [apply_fn(s, weight[c], total, hidden, eps) for (s, _), c in zip(parts, cols)]
    return torch.cat(ys, -1), torch.cat([s for s, _ in parts], -1)


def rmsnorm_tp(
    x: torch.Tensor,
    residual: torch.Tensor | None,
    weight: torch.Tensor,
    hidden: int,
    eps: float = 1e-6,
    *,
    group=None,
    partial_fn: Callable = rmsnorm_shard_partial_hip,
    apply_fn: Callable = rmsnorm_shard_apply_hip,
) -> tuple[torch.Tensor, torch.Tensor]:
    """This rank's slice of ``(rmsnorm(x + residual), x + residual)`` in a
    ``torch.distributed`` group whose ranks hold the column slices of every row.

    ``x``, ``residual`` and ``weight`` are the rank's slices; ``hidden`` is the
    full row length. The per-row partial sums of squares (one fp32 per row) are
    summed over the group with one all-reduce. Over RCCL (backend ``"nccl"``)
    the device tensor is reduced in place; gloo gets a host copy, made and
    copied back synchronously, since gloo is given CPU tensors only.
    """
    import torch.distributed as dist

    if weight.shape[-1] != x.shape[-1]:
        raise ValueError(f"weight slice {tuple(weight.shape)} does not match x slice {tuple(x.shape)}")
    s, partial = partial_fn(x, residual)
    if partial.is_cuda and dist.get_backend(group) == "gloo":
        host = partial.cpu()
        dist.all_reduce(host, op=dist.ReduceOp.SUM, group=group)
        partial.copy_(host)
    else:
        dist.all_reduce(partial, op=dist.ReduceOp.SUM, group=group)
    return apply_fn(s, weight, partial, hidden, eps), s


__all__ = [
    "rmsnorm_sharded",
    "rmsnorm_tp",
    "rmsnorm_shard_apply_hip",
    "rmsnorm_shard_apply_ref",
    "rmsnorm_shard_partial_hip",
    "rmsnorm_shard_partial_ref",
]
