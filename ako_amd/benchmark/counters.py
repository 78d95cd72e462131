"""Launch driver for rocprofv3 counter passes over the hot-path cells.

Run under ``rocprofv3 --pmc FETCH_SIZE`` (then ``--pmc WRITE_SIZE``): it
builds every input first, then launches each cell ``--repeat`` times back to
back, in the fixed order of ``CELLS``, and finally a plain elementwise kernel
of known traffic (``torch.neg`` over 1 GiB of fp16: reads 1 GiB, writes
1 GiB) whose counter reading gives the scale factor between the counters and
true HBM bytes on this device. ``ako_amd.benchmark.rocprof`` matches the
dispatches back to cells by that order.

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -o fetch -- \\
        python -m ako_amd.benchmark.counters --manifest OUT/manifest.json
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch

from ako_amd.benchmark import roofline as rf
from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
from ako_amd.ops.rmsnorm_tp import rmsnorm_shard_apply_hip, rmsnorm_shard_partial_hip
from ako_amd.ops.rope_hip import rope_hip, rope_qk_cache_hip, rope_qk_hip
from ako_amd.ops.rope_ref import build_rope_tables
from ako_amd.ops.swiglu_hip import swiglu_hip

REFERENCE_BYTES = 1 << 30


def build(device: torch.device):
    gen = torch.Generator(device=device).manual_seed(0)

    def rnd(*shape, dtype, scale=1.0, shift=0.0):
        return (torch.randn(*shape, generator=gen, device=device) * scale + shift).to(dtype)

    cells = []
    for dtype, tag in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        for h in (4096, 8192, 16384):
            x, r = rnd(16384, h, dtype=dtype), rnd(16384, h, dtype=dtype)
            w = rnd(h, dtype=dtype, scale=0.1, shift=1.0)
            cells.append((f"rmsnorm_{tag}_16384x{h}", rf.alg_bytes_rmsnorm(16384, h, dtype),
                          lambda x=x, w=w: rmsnorm_hip(x, w, 1e-6)))
            cells.append((f"rmsnorm_residual_{tag}_16384x{h}", rf.alg_bytes_rmsnorm_residual(16384, h, dtype),
                          lambda x=x, r=r, w=w: rmsnorm_residual_hip(x, r, w, 1e-6)))
        cos, sin = build_rope_tables(2048, 128, device=device)
        cos, sin = cos.to(dtype), sin.to(dtype)
        q, k = rnd(4, 2048, 32, 128, dtype=dtype), rnd(4, 2048, 8, 128, dtype=dtype)
        cells.append((f"rope_q_{tag}_4x2048x32x128", rf.alg_bytes_rope(4, 2048, 32, 128, dtype, dtype),
                      lambda q=q, c=cos, s=sin: rope_hip(q, c, s)))
        cells.append((f"rope_qk_{tag}_4x2048", rf.alg_bytes_rope(4, 2048, 40, 128, dtype, dtype),
                      lambda q=q, k=k, c=cos, s=sin: rope_qk_hip(q, k, c, s)))
        # q, k and v of a 2048-token prefill into a heads-major KV cache at slot 0.
        v = rnd(4, 2048, 8, 128, dtype=dtype)
        kc, vc = rnd(4, 8, 2048, 128, dtype=dtype), rnd(4, 8, 2048, 128, dtype=dtype)
        pos = torch.zeros(1, dtype=torch.long, device=device)
        cells.append((f"rope_qk_cache_{tag}_4x2048_q32_kv8",
                      rf.alg_bytes_rope_qk_cache(4, 2048, 32, 8, 128, dtype, dtype),
                      lambda q=q, k=k, v=v, c=cos, s=sin, kc=kc, vc=vc, p=pos:
                      rope_qk_cache_hip(q, k, v, c, s, p, kc, vc)))
        # One TP=8 rank's slice of the widest configs[1] row.
        xs, rs = rnd(16384, 2048, dtype=dtype), rnd(16384, 2048, dtype=dtype)
        ws = rnd(2048, dtype=dtype, scale=0.1, shift=1.0)
        total = torch.full((16384,), 2048.0, device=device)
        cells.append((f"rmsnorm_shard_partial_{tag}_16384x2048_residual",
                      rf.alg_bytes_rmsnorm_shard_partial(16384, 2048, dtype, residual=True),
                      lambda x=xs, r=rs: rmsnorm_shard_partial_hip(x, r)))
        cells.append((f"rmsnorm_shard_apply_{tag}_16384x2048", rf.alg_bytes_rmsnorm_shard_apply(16384, 2048, dtype),
                      lambda x=xs, w=ws, t=total: rmsnorm_shard_apply_hip(x, w, t, 16384, 1e-6)))
    g, u = rnd(16384, 14336, dtype=torch.bfloat16), rnd(16384, 14336, dtype=torch.bfloat16)
    cells.append(("swiglu_bf16_16384x14336", rf.alg_bytes_swiglu(16384, 14336, torch.bfloat16),
                  lambda g=g, u=u: swiglu_hip(g, u)))
    src = torch.ones(REFERENCE_BYTES // 2, dtype=torch.float16, device=device)
    dst = torch.empty_like(src)
    reference = ("reference_neg_fp16_1GiB", 2 * REFERENCE_BYTES, lambda: torch.neg(src, out=dst))
    return cells, reference


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--repeat", type=int, default=3)
    ap.add_argument("--manifest", type=Path, required=True)
    args = ap.parse_args(argv)
    device = torch.device("cuda", 0)
    cells, reference = build(device)
    torch.cuda.synchronize()
    order = []
    for name, nbytes, fn in cells + [reference]:
        for _ in range(args.repeat):
            fn()
            order.append({"cell": name, "alg_bytes": nbytes})
        torch.cuda.synchronize()
    args.manifest.parent.mkdir(parents=True, exist_ok=True)
    args.manifest.write_text(json.dumps({"repeat": args.repeat, "dispatches": order}, indent=1))
    print(f"launched {len(order)} dispatches", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
