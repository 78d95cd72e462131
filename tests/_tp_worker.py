"""One rank of the multi-process RMSNorm-over-slices tests (spawned by
``tests/test_rmsnorm_tp.py``): joins a gloo group on 127.0.0.1, takes its
column slice of seeded full-size inputs, runs ``rmsnorm_tp`` and saves its
output slices for the parent to check."""

from __future__ import annotations

from pathlib import Path


def rank_main(rank: int, world: int, port: int, out_dir: str, device: str, dtype_name: str,
              rows: int, hidden: int, use_hip: bool) -> None:
    import torch
    import torch.distributed as dist

    from ako_amd.ops.rmsnorm_tp import (
        rmsnorm_shard_apply_hip,
        rmsnorm_shard_apply_ref,
        rmsnorm_shard_partial_hip,
        rmsnorm_shard_partial_ref,
        rmsnorm_tp,
    )

    import datetime

    # A bounded rendezvous and collective timeout: a rank that fails ends the
    # test instead of leaving the other waiting for gloo's 30-minute default.
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank, world_size=world,
                            timeout=datetime.timedelta(seconds=60))
    try:
        dtype = getattr(torch, dtype_name)
        x, r, w = full_inputs(rows, hidden, dtype)
        width = hidden // world
        cols = slice(rank * width, (rank + 1) * width)
        dev = torch.device(device)
        xs, rs, ws = (t[..., cols].contiguous().to(dev) for t in (x, r, w))
        fns = (dict(partial_fn=rmsnorm_shard_partial_hip, apply_fn=rmsnorm_shard_apply_hip) if use_hip
               else dict(partial_fn=rmsnorm_shard_partial_ref, apply_fn=rmsnorm_shard_apply_ref))
        y, s = rmsnorm_tp(xs, rs, ws, hidden, 1e-6, **fns)
        yp, sp = rmsnorm_tp(xs, None, ws, hidden, 1e-6, **fns)
        torch.save({"y": y.cpu(), "s": s.cpu(), "y_plain": yp.cpu()}, Path(out_dir) / f"rank{rank}.pt")
    finally:
        dist.destroy_process_group()


def full_inputs(rows: int, hidden: int, dtype):
    """The seeded full rows every rank slices (x, residual ~N(0,1), weight ~N(1,0.1))."""
    import torch

    g = torch.Generator().manual_seed(11)
    x = torch.randn(rows, hidden, generator=g).to(dtype)
    r = torch.randn(rows, hidden, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype)
    return x, r, w
