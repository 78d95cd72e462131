#!/usr/bin/env python
"""Headline benchmark: achieved HBM bandwidth of the HIP RMSNorm kernels.

One *step* is one pass of the hot path over the BASELINE.json configs[1]
prefill grid: plain RMSNorm and residual-add RMSNorm, fp16 and bf16, hidden
4096 / 8192 / 16384, 16384 rows (12 kernel launches, 11.27 GB of algorithmic
traffic). Inputs are resident in HBM before timing starts. Every launch of a
step reads buffers of its own (the plain and the residual launch of a width
do not share x), 11 GB per step against a 256 MB Infinity Cache, so every
launch reads cold data. ``value`` is algorithmic bytes per step x steps /
elapsed device time, in GB/s.

The printed line (one JSON object, kept under 8 KB) also carries:
  roofline      the dominant kernel (the slowest launch of the step) with its
                per-launch duration from HIP events on the launch stream,
                bound to each launch's dispatch (the kernel's own start and
                end, no marker packets between launches), and a plain device
                copy of the same byte count timed the same way
                (copy_same_bytes: what the plainest stream of those bytes
                reaches; a reference, which a kernel can pass);
  cpu_baseline  the reference's unfused PyTorch path on host CPU tensors with
                all of torch's threads: RMSNorm on the step's own 12 cells at
                full size (the lead figure), RoPE q+k at (4, 2048) and SwiGLU
                at M = 4096, each the median of its passes with the slowest
                and fastest; the numpy oracle on one thread beside the RMSNorm
                figure, on a 64-row sample;
  selection     the reference's selection (gate + timing + cache record) run
                here over the configs[1]-[3] grid, decode cells included: how
                many cells the HIP candidate won, and its largest ulp error
                per op;
  decoder       configs[4]: the 4-layer fp16 decoder, prefill 512 tokens then
                128 greedy steps, eager PyTorch vs the dispatcher, each also
                with decode steps replayed from a HIP graph;
  rope_prefill  RoPE at (4, 2048) as the fused q+k launch, and as the
                decoder's own prefill call, which also writes k and v into
                its KV cache (qk_cache); back to back, and per launch with
                launch-bound events (per_launch: the kernel's own duration);
  prefill_floor per op, the prefill cell with the lowest share of peak,
                timed back to back, and the lowest per launch.

Every timed cell goes to ``--cells-out`` (reports/mi355x/bench_cells.json by
default) in the reference's report layout, with the selection's rows:
  per_kernel    every launch of the step, each beside its copy ceiling, by
                launch-bound events (as the roofline) and, under back_to_back,
                on its own as 60 launches between one event pair over cold
                input copies, beside a copy timed the same way;
  extras        the RoPE and SwiGLU cells, the
                decode-size RMSNorm cells, the KV-cache RoPE and the
                tensor-parallel RMSNorm halves; streaming cells back to back
                and per launch (launch-bound events over three passes of
                their cold input copies), each beside the copy timed the same
                way, decode cells as graph-replayed device time with inputs
                hot (graph_us) and in no cache (graph_cold_us).

``dtype`` is the arithmetic type of the kernels (fp32); the stored tensors
are fp16 and bf16 (``config.storage_dtypes``).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras]
       [--no-selection] [--no-decoder] [--no-cpu] [--cells-out PATH]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

RMS_HIDDEN = (4096, 8192, 16384)
RMS_ROWS = 16384
#: Cells at least this large are streaming cells, reported beside a copy of the same bytes.
STREAMING_BYTES = 16 * 2**20


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-extras", action="store_true", help="skip the RoPE/SwiGLU/decode cells")
    ap.add_argument("--no-selection", action="store_true", help="skip the selection over the grid")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decoder", action="store_true", help="skip the configs[4] decoder run")
    ap.add_argument("--cpu-seconds", type=float, default=16.0,
                    help="host time the CPU baseline may take, over all its figures")
    ap.add_argument("--cells-out", type=Path, default=ROOT / "reports" / "mi355x" / "bench_cells.json",
                    help="where every timed cell and the selection rows are written (report layout)")
    ap.add_argument("--traffic", type=Path, default=ROOT / "profiles" / "hbm_traffic_hot_path_cells.md",
                    help="rocprofv3 FETCH/WRITE summary (ako_amd.benchmark.rocprof) for the kernels")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class CopyCeilings:
    """Copy-of-the-same-bytes figures by byte count, each measured once."""

    def __init__(self, rf) -> None:
        self.rf = rf
        self.seen: dict[int, dict | None] = {}

    def get(self, alg_bytes: int) -> dict | None:
        if alg_bytes not in self.seen:
            self.seen[alg_bytes] = self.rf.copy_same_bytes(alg_bytes)
        return self.seen[alg_bytes]

    def annotate(self, row: dict, gbps: float, *, back_to_back: bool = False) -> None:
        """Add the copy's share of peak and the kernel's rate over the copy's,
        the copy timed the way the row was (launch-bound events, or one event
        pair around back-to-back launches)."""
        copy = self.get(row["alg_bytes"])
        if copy is None:
            return
        if back_to_back and "best_b2b_gbps" in copy:
            row["copy_pct_hbm_peak"] = round(100 * copy["best_b2b_frac"], 2)
            row["kernel_over_copy"] = round(gbps / copy["best_b2b_gbps"], 4)
        elif not back_to_back:
            row["copy_pct_hbm_peak"] = round(100 * copy["frac"], 2)
            row["kernel_over_copy"] = round(gbps / copy["gbps"], 4)


def headline(args, torch, rf, dev, peak, rnd):
    """The metric's workload: configs[1] prefill grid, 12 launches per step."""
    from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip

    calls = []
    for dtype in (torch.float16, torch.bfloat16):
        tag = "fp16" if dtype == torch.float16 else "bf16"
        for h in RMS_HIDDEN:
            x_plain = rnd(RMS_ROWS, h, dtype=dtype)
            x_res = rnd(RMS_ROWS, h, dtype=dtype)
            r = rnd(RMS_ROWS, h, dtype=dtype)
            w = rnd(h, dtype=dtype, scale=0.1, shift=1.0)
            calls.append((f"rmsnorm_{tag}_{RMS_ROWS}x{h}", rf.alg_bytes_rmsnorm(RMS_ROWS, h, dtype),
                          lambda x=x_plain, w=w: rmsnorm_hip(x, w, 1e-6)))
            calls.append((f"rmsnorm_residual_{tag}_{RMS_ROWS}x{h}",
                          rf.alg_bytes_rmsnorm_residual(RMS_ROWS, h, dtype),
                          lambda x=x_res, r=r, w=w: rmsnorm_residual_hip(x, r, w, 1e-6)))
    bytes_per_step = sum(b for _, b, _ in calls)
    log(f"workload: {len(calls)} launches/step, {bytes_per_step / 1e9:.3f} GB/step, "
        f"warmup {args.warmup}, steps {args.steps}")
    rf.warm(calls, args.warmup)
    total_ms = rf.time_steps(calls, steps=args.steps)
    # The dominant kernel's launch duration: the same K steps again, now with an
    # event pair bound to every launch (hipExtLaunchKernelGGL through
    # ako_time_next_launch: each pair holds its kernel's own start and end).
    per_launch = rf.time_each_launch(calls, steps=args.steps, kernel_events=True)
    del calls
    torch.cuda.empty_cache()
    return bytes_per_step, total_ms, per_launch


def headline_back_to_back(torch, rf, dev, rnd) -> dict[str, float]:
    """Each cell of the step on its own: mean ms per launch over 60 launches
    queued back to back between one event pair, cycling through enough input
    copies that every launch reads cold data (no per-launch events, whose
    1.5-2 us would be counted in the launch); the median of three such runs
    after two discarded ones (``roofline.settled_back_to_back``)."""
    from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip

    out = {}
    for dtype in (torch.float16, torch.bfloat16):
        tag = "fp16" if dtype == torch.float16 else "bf16"
        for h in RMS_HIDDEN:
            w = rnd(h, dtype=dtype, scale=0.1, shift=1.0)
            for residual in (False, True):
                nbytes = (rf.alg_bytes_rmsnorm_residual(RMS_ROWS, h, dtype) if residual
                          else rf.alg_bytes_rmsnorm(RMS_ROWS, h, dtype))
                n = rf.copies_for_cold(nbytes, dev)
                sets = [(rnd(RMS_ROWS, h, dtype=dtype), rnd(RMS_ROWS, h, dtype=dtype) if residual else None)
                        for _ in range(n)]
                fns = [(lambda x=x, r=r: rmsnorm_residual_hip(x, r, w, 1e-6)) if residual
                       else (lambda x=x: rmsnorm_hip(x, w, 1e-6)) for x, r in sets]
                for fn in fns:
                    fn()
                name = f"rmsnorm{'_residual' if residual else ''}_{tag}_{RMS_ROWS}x{h}"
                out[name] = rf.settled_back_to_back(fns, launches=60)
                del sets, fns
                torch.cuda.empty_cache()
    return out


def extras_cells(torch, rf, dev, rnd):
    """(name, alg_bytes, [thunks over input copies], decode) for every extra cell."""
    from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
    from ako_amd.ops.rmsnorm_tp import rmsnorm_shard_apply_hip, rmsnorm_shard_partial_hip
    from ako_amd.ops.rope_hip import rope_hip, rope_qk_cache_hip, rope_qk_hip
    from ako_amd.ops.rope_ref import build_rope_tables
    from ako_amd.ops.swiglu_hip import swiglu_hip

    cells = []

    def add(name, nbytes, make, copies, decode):
        cells.append((name, nbytes, [make(i) for i in range(copies)], decode))

    decode_copies = 64  # independent inputs for the cold graph (one per call)
    for dtype in (torch.float16, torch.bfloat16):
        tag = "fp16" if dtype == torch.float16 else "bf16"
        for b, s in ((4, 2048), (64, 1), (1, 1)):
            cos, sin = build_rope_tables(s, 128, device=dev)
            cos, sin = cos.to(dtype), sin.to(dtype)
            decode = s == 1
            n = decode_copies if decode else rf.copies_for_cold(rf.alg_bytes_rope(b, s, 40, 128, dtype, dtype), dev)
            qs = [rnd(b, s, 32, 128, dtype=dtype) for _ in range(n)]
            ks = [rnd(b, s, 8, 128, dtype=dtype) for _ in range(n)]
            add(f"rope_q_{tag}_{b}x{s}x32x128", rf.alg_bytes_rope(b, s, 32, 128, dtype, dtype),
                lambda i, c=cos, sn=sin, qs=qs: (lambda q=qs[i]: rope_hip(q, c, sn, "neox")), n, decode)
            add(f"rope_k_{tag}_{b}x{s}x8x128", rf.alg_bytes_rope(b, s, 8, 128, dtype, dtype),
                lambda i, c=cos, sn=sin, ks=ks: (lambda k=ks[i]: rope_hip(k, c, sn, "neox")), n, decode)
            add(f"rope_qk_{tag}_{b}x{s}", rf.alg_bytes_rope(b, s, 40, 128, dtype, dtype),
                lambda i, c=cos, sn=sin, qs=qs, ks=ks: (lambda q=qs[i], k=ks[i]: rope_qk_hip(q, k, c, sn, "neox")),
                n, decode)
            if (b, s) == (4, 2048):
                # The decoder's prefill call: q rotated, k rotated and v copied
                # into heads-major KV caches at slot 0, one launch per copy,
                # each copy with caches of its own.
                nb = rf.alg_bytes_rope_qk_cache(b, s, 32, 8, 128, dtype, dtype)
                nc = rf.copies_for_cold(nb, dev)
                vs = [rnd(b, s, 8, 128, dtype=dtype) for _ in range(nc)]
                caches = [(torch.empty(b, 8, s, 128, dtype=dtype, device=dev),
                           torch.empty(b, 8, s, 128, dtype=dtype, device=dev)) for _ in range(nc)]
                pos0 = torch.zeros(1, dtype=torch.long, device=dev)
                add(f"rope_qk_cache_{tag}_{b}x{s}_q32_kv8", nb,
                    lambda i, c=cos, sn=sin, qs=qs, ks=ks, vs=vs, caches=caches, p=pos0:
                        (lambda q=qs[i % len(qs)], k=ks[i % len(ks)], v=vs[i], kv=caches[i]:
                         rope_qk_cache_hip(q, k, v, c, sn, p, kv[0], kv[1], "neox")),
                    nc, False)
    # configs[4] decode step, one layer: RoPE of q and k plus the KV-cache
    # append, fused (one launch) and as the unfused sequence it replaces.
    dtype = torch.float16
    full_cos, full_sin = build_rope_tables(640, 128, device=dev)
    qkv = [tuple(rnd(1, 1, 32, 128, dtype=dtype) for _ in range(3)) for _ in range(decode_copies)]
    kc, vc = rnd(1, 32, 640, 128, dtype=dtype), rnd(1, 32, 640, 128, dtype=dtype)
    pos = torch.full((1,), 511, dtype=torch.long, device=dev)
    cache_bytes = rf.alg_bytes_rope_qk_cache(1, 1, 32, 32, 128, dtype, torch.float32)

    def unfused(i):
        q1, k1, v1 = qkv[i]

        def step():
            c, sn = full_cos.index_select(0, pos), full_sin.index_select(0, pos)
            qo, ko = rope_qk_hip(q1, k1, c, sn, "neox")
            kc.index_copy_(2, pos, ko.transpose(1, 2))
            vc.index_copy_(2, pos, v1.transpose(1, 2))
            return qo
        return step

    add("rope_qk_cache_fp16_1x1_q32_kv32_slot511of640", cache_bytes,
        lambda i: (lambda t=qkv[i]: rope_qk_cache_hip(t[0], t[1], t[2], full_cos, full_sin, pos, kc, vc, "neox")),
        decode_copies, True)
    add("rope_qk_then_index_copy_fp16_1x1_q32_kv32", cache_bytes, unfused, decode_copies, True)
    # One tensor-parallel rank's slice of the widest configs[1] row (TP=8:
    # 2048 of 16384): residual + partial sum of squares, then the apply half.
    for dtype in (torch.float16, torch.bfloat16):
        tag = "fp16" if dtype == torch.float16 else "bf16"
        rows_tp, shard = RMS_ROWS, 2048
        nb_p = rf.alg_bytes_rmsnorm_shard_partial(rows_tp, shard, dtype, residual=True)
        nb_a = rf.alg_bytes_rmsnorm_shard_apply(rows_tp, shard, dtype)
        n = rf.copies_for_cold(nb_p, dev)
        xs = [rnd(rows_tp, shard, dtype=dtype) for _ in range(n)]
        rs = [rnd(rows_tp, shard, dtype=dtype) for _ in range(n)]
        w_tp = rnd(shard, dtype=dtype, scale=0.1, shift=1.0)
        tot = torch.full((rows_tp,), float(shard), device=dev)
        add(f"rmsnorm_shard_partial_{tag}_{rows_tp}x{shard}_residual", nb_p,
            lambda i, xs=xs, rs=rs: (lambda x=xs[i], r=rs[i]: rmsnorm_shard_partial_hip(x, r)), n, False)
        add(f"rmsnorm_shard_apply_{tag}_{rows_tp}x{shard}", nb_a,
            lambda i, xs=xs, w=w_tp, t=tot, shard=shard:
                (lambda s_=xs[i]: rmsnorm_shard_apply_hip(s_, w, t, 8 * shard, 1e-6)), n, False)
    for m in (16384, 4096, 256, 16, 1):
        dtype = torch.bfloat16
        nbytes = rf.alg_bytes_swiglu(m, 14336, dtype)
        decode = m <= 16
        n = decode_copies if decode else rf.copies_for_cold(nbytes, dev)
        gs = [rnd(m, 14336, dtype=dtype) for _ in range(n)]
        us = [rnd(m, 14336, dtype=dtype) for _ in range(n)]
        add(f"swiglu_bf16_{m}x14336", nbytes, lambda i, gs=gs, us=us: (lambda g=gs[i], u=us[i]: swiglu_hip(g, u)),
            n, decode)
    for dtype in (torch.float16, torch.bfloat16):
        tag = "fp16" if dtype == torch.float16 else "bf16"
        for rows in (1, 32):
            for h in RMS_HIDDEN:
                sets = [(rnd(rows, h, dtype=dtype), rnd(rows, h, dtype=dtype),
                         rnd(h, dtype=dtype, scale=0.1, shift=1.0)) for _ in range(decode_copies)]
                add(f"rmsnorm_{tag}_{rows}x{h}", rf.alg_bytes_rmsnorm(rows, h, dtype),
                    lambda i, sets=sets: (lambda t=sets[i]: rmsnorm_hip(t[0], t[2], 1e-6)), decode_copies, True)
                add(f"rmsnorm_residual_{tag}_{rows}x{h}", rf.alg_bytes_rmsnorm_residual(rows, h, dtype),
                    lambda i, sets=sets: (lambda t=sets[i]: rmsnorm_residual_hip(t[0], t[1], t[2], 1e-6)),
                    decode_copies, True)
    return cells


def per_launch_row(name, nbytes, fns, rf, peak, ceilings) -> dict | None:
    """A streaming cell's launches timed one by one with events bound to each
    launch (the kernel's own duration, as the roofline is timed), three
    passes over its cold input copies, beside the copy's per-launch figure.
    None when a call makes no launch through the library."""
    calls = [(name, nbytes, fn) for fn in fns]
    try:
        stats = rf.time_each_launch(calls, steps=3, lead_passes=1, kernel_events=True)[0]
    except RuntimeError as err:
        log(f"{name}: no launch-bound timing ({err})")
        return None
    out = {"mean_us": round(stats.mean_ms * 1e3, 3), "launches": len(stats.durations_ms),
           "pct_hbm_peak": round(100.0 * stats.gbps() / peak, 2)}
    copy = ceilings.get(nbytes)
    if copy is not None:
        out["copy_pct_hbm_peak"] = round(100 * copy["frac"], 2)
        out["kernel_over_copy"] = round(stats.gbps() / copy["gbps"], 4)
    return out


def time_extras(cells, torch, rf, peak, ceilings):
    """Each cell: 60 back-to-back launches over its input copies between one
    event pair (per-launch events would distort 5-30 us kernels; streaming
    cells take the median of three such timings) beside the copy of the same
    bytes; decode cells also as device time per call from replayed HIP graphs,
    inputs hot (64 calls on one input) and cold (64 calls on 64 inputs after
    an eviction pass)."""
    extras = []
    for _, _, fns, _ in cells:
        for fn in fns[:2]:
            fn()
    torch.cuda.synchronize()
    for name, nbytes, fns, decode in cells:
        if decode:
            ms = rf.time_back_to_back(fns[:1], launches=60)  # hot: one input, as before
        else:
            # Median of three settled timings: single 60-launch timings of
            # these 8-220 us launches move by several percent from one to the next.
            ms = rf.settled_back_to_back(fns, launches=60)
        stats = rf.LaunchStats(name, nbytes, [ms])
        row = stats.to_dict(peak)
        row.pop("launches")
        row.pop("p50_us")
        row["copies"] = 1 if decode else len(fns)
        if nbytes >= STREAMING_BYTES:
            ceilings.annotate(row, stats.gbps(), back_to_back=True)
            row["per_launch"] = per_launch_row(name, nbytes, fns, rf, peak, ceilings)
        if decode:
            # Median of five graph timings: one is under a millisecond of
            # device time, and clock changes move single readings by up to 15%.
            row["graph_us"] = round(sorted(rf.time_graph_replay(fns[0]) for _ in range(5))[2], 3)
            row["graph_cold_us"] = round(rf.time_graph_cold(fns), 3)
        extras.append(row)
    return extras


#: Library calls per graph-replayed configs[4] decode step: an input and a
#: post-attention residual norm per layer (layer 0's input norm is plain, and
#: the final norm is a residual one), RoPE with the cache append per layer,
#: SwiGLU per layer.
DECODE_STEP_CALLS = {"rmsnorm": 1, "rmsnorm_residual": 8, "rope_qk_cache": 4, "swiglu": 4}


def in_model_decode(torch, rf, dev, rnd):
    """configs[4]'s decode calls as the model runs them: each right behind
    the fp16 GEMV that writes its input (graph_in_model_us, from
    ``time_graph_after_producer``), beside the same call on cold inputs with
    no producer (graph_cold_us). The producers are the model's own
    projections at batch 1: o_proj (4096 -> 4096) ahead of the residual
    norm, the fused qkv projection (4096 -> 12288) ahead of RoPE + cache
    append, gate and up (4096 -> 11008 each) ahead of SwiGLU; every pair has
    its own weights, so a pass over the pairs streams 1-3 GB and each call
    finds its inputs, and its own code, as the model leaves them."""
    from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
    from ako_amd.ops.rope_hip import rope_qk_cache_hip
    from ako_amd.ops.rope_ref import build_rope_tables
    from ako_amd.ops.swiglu_hip import swiglu_hip

    dt = torch.float16
    h, heads, d, ffn, slots = 4096, 32, 128, 11008, 640
    out = {}

    def gemv(n_out):
        a = rnd(1, h, dtype=dt)
        w = rnd(n_out, h, dtype=dt, scale=0.02)
        y = torch.empty(1, n_out, dtype=dt, device=dev)
        return a, w, y

    def run(name, pairs):
        calls = [c for _, c in pairs]
        in_model = rf.time_graph_after_producer(pairs)
        cold = rf.time_graph_cold(calls)
        out[name] = {"graph_in_model_us": round(in_model, 3), "graph_cold_us": round(cold, 3),
                     "per_step": DECODE_STEP_CALLS[name]}

    sets = []
    for _ in range(32):
        a, w, x = gemv(h)
        sets.append((lambda a=a, w=w, x=x: torch.mm(a, w.t(), out=x), x, rnd(1, h, dtype=dt),
                     rnd(h, dtype=dt, scale=0.1, shift=1.0)))
    run("rmsnorm_residual", [(p, lambda x=x, r=r, nw=nw: rmsnorm_residual_hip(x, r, nw, 1e-6))
                             for p, x, r, nw in sets])
    run("rmsnorm", [(p, lambda x=x, nw=nw: rmsnorm_hip(x, nw, 1e-6)) for p, x, _, nw in sets])
    del sets
    torch.cuda.empty_cache()

    cos, sin = build_rope_tables(slots, d, device=dev)
    pos = torch.full((1,), 511, dtype=torch.long, device=dev)
    pairs = []
    for _ in range(16):
        a, w, qkv = gemv(3 * h)
        q = qkv[:, :h].view(1, 1, heads, d)
        k = qkv[:, h:2 * h].view(1, 1, heads, d)
        v = qkv[:, 2 * h:].view(1, 1, heads, d)
        kc = torch.zeros(1, heads, slots, d, dtype=dt, device=dev)
        vc = torch.zeros(1, heads, slots, d, dtype=dt, device=dev)
        pairs.append((lambda a=a, w=w, y=qkv: torch.mm(a, w.t(), out=y),
                      lambda q=q, k=k, v=v, kc=kc, vc=vc: rope_qk_cache_hip(q, k, v, cos, sin, pos, kc, vc, "neox")))
    run("rope_qk_cache", pairs)
    del pairs
    torch.cuda.empty_cache()

    pairs = []
    for _ in range(16):
        a = rnd(1, h, dtype=dt)
        wg, wu = rnd(ffn, h, dtype=dt, scale=0.02), rnd(ffn, h, dtype=dt, scale=0.02)
        g, u = torch.empty(1, ffn, dtype=dt, device=dev), torch.empty(1, ffn, dtype=dt, device=dev)

        def produce(a=a, wg=wg, wu=wu, g=g, u=u):
            torch.mm(a, wg.t(), out=g)
            torch.mm(a, wu.t(), out=u)
        pairs.append((produce, lambda g=g, u=u: swiglu_hip(g, u)))
    run("swiglu", pairs)
    del pairs
    torch.cuda.empty_cache()
    total = sum(v["graph_in_model_us"] * v["per_step"] for v in out.values())
    cold = sum(v["graph_cold_us"] * v["per_step"] for v in out.values())
    return {"ops": out, "step_library_us": round(total, 1), "step_library_cold_us": round(cold, 1),
            "calls_per_step": sum(DECODE_STEP_CALLS.values())}


def _per_launch_brief(row: dict) -> dict | None:
    per = row.get("per_launch")
    if not per:
        return None
    return {k: per[k] for k in ("pct_hbm_peak", "kernel_over_copy") if k in per}


def rope_prefill_summary(extras, ceilings):
    """RoPE at the prefill shape: q and k in one launch (configs[2]'s pair),
    and the decoder's own call, which also writes k and v into the KV cache."""
    by_name = {r["name"]: r for r in extras}
    out = {}
    for tag in ("fp16", "bf16"):
        qk = by_name.get(f"rope_qk_{tag}_4x2048")
        k = by_name.get(f"rope_k_{tag}_4x2048x8x128")
        cache = by_name.get(f"rope_qk_cache_{tag}_4x2048_q32_kv8")
        if qk is None:
            continue
        out[tag] = {"cell": qk["name"], "pct_hbm_peak": qk["pct_hbm_peak"],
                    "copy_pct_hbm_peak": qk.get("copy_pct_hbm_peak"), "kernel_over_copy": qk.get("kernel_over_copy"),
                    "per_launch": _per_launch_brief(qk)}
        if cache is not None:
            out[tag]["qk_cache"] = {"pct_hbm_peak": cache["pct_hbm_peak"],
                                    "copy_pct_hbm_peak": cache.get("copy_pct_hbm_peak"),
                                    "kernel_over_copy": cache.get("kernel_over_copy"),
                                    "per_launch": _per_launch_brief(cache)}
        if k is not None:
            out[tag]["k_alone"] = {"pct_hbm_peak": k["pct_hbm_peak"], "copy_pct_hbm_peak": k.get("copy_pct_hbm_peak"),
                                   "note": "34 MB launch: a copy of that size reaches little more"}
    return out


def selection(torch):
    """The reference's Algorithm 1 over the configs[1]-[3] grid on this GPU."""
    from ako_amd.benchmark.sweep import run

    with tempfile.TemporaryDirectory(prefix="ako-selection-") as tmp:
        summary = run(Path(tmp), {"rmsnorm", "rmsnorm_residual", "rope", "rope_qk", "swiglu"},
                      warmup=5, repeats=20, quiet=True)
        rows = []
        for report in sorted(Path(tmp).glob("selection_*.json")):
            if report.name == "selection_summary.json":
                continue
            data = json.loads(report.read_text())
            rows += [{"operation": data["operation"], **row} for row in data["comparisons"]]
    summary["win_rate"] = summary.pop("hip_win_rate")
    torch.cuda.empty_cache()
    return summary, rows


def _timed_passes(cells, seconds: float, min_passes: int = 3) -> list[float]:
    """Seconds per pass over ``cells`` (one untimed pass first), passes
    repeated until ``seconds`` have gone by and at least ``min_passes`` ran."""
    for fn in cells:
        fn()
    times, t_start = [], time.perf_counter()
    while True:
        t0 = time.perf_counter()
        for fn in cells:
            fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start >= seconds and len(times) >= min_passes:
            return times


def _rate(nbytes: int, times: list[float]) -> dict:
    """Median GB/s over the passes, with the slowest and fastest pass."""
    rates = sorted(nbytes / t / 1e9 for t in times)
    return {"value": round(statistics.median(rates), 3), "spread": [round(rates[0], 3), round(rates[-1], 3)],
            "passes": len(times)}


def cpu_baseline(args, torch, rf, value):
    """The reference's unfused PyTorch path on the host cores: every op of
    the metric, on host CPU tensors with all of torch's threads. RMSNorm (the
    lead figure) on the step's own 12 cells at full size, RoPE q+k at
    (4, 2048) and SwiGLU at M = 4096, each the median of its timed passes
    with the slowest and fastest pass; the numpy oracle on one thread beside
    the RMSNorm figure, on a row sample."""
    import numpy as np

    from ako_amd.ops.rmsnorm_ref import rmsnorm_ref, rmsnorm_residual_ref
    from ako_amd.ops.rope_ref import build_rope_tables, rope_ref
    from ako_amd.ops.swiglu_ref import swiglu_ref
    from oracle import ops as oracle

    def storage(t):
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16)
        return t.numpy()

    budget = args.cpu_seconds
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    # One pool of N(0,1) values; each cell's x and residual are windows of it
    # at different offsets (drawing 2.8e9 fresh values would take longer than
    # the timing itself).
    widest = max(RMS_HIDDEN)
    pool = torch.randn(RMS_ROWS * widest + 2 * widest, generator=g)
    rms_cells, rms_bytes, port_cells, port_bytes = [], 0, [], 0
    port_rows = 64
    for dtype in (torch.float16, torch.bfloat16):
        name = "float16" if dtype == torch.float16 else "bfloat16"
        for i, h in enumerate(RMS_HIDDEN):
            n = RMS_ROWS * h
            x = pool[i:i + n].view(RMS_ROWS, h).to(dtype)
            r = pool[widest + i:widest + i + n].view(RMS_ROWS, h).to(dtype)
            w = (torch.randn(h, generator=g) * 0.1 + 1.0).to(dtype)
            rms_cells += [lambda x=x, w=w: rmsnorm_ref(x, w, 1e-6),
                          lambda x=x, r=r, w=w: rmsnorm_residual_ref(x, r, w, 1e-6)]
            rms_bytes += rf.alg_bytes_rmsnorm(RMS_ROWS, h, dtype) + rf.alg_bytes_rmsnorm_residual(RMS_ROWS, h, dtype)
            xn, rn, wn = storage(x[:port_rows]), storage(r[:port_rows]), storage(w)
            port_cells += [lambda xn=xn, wn=wn, name=name: oracle.rmsnorm(xn, wn, 1e-6, dtype=name),
                           lambda xn=xn, rn=rn, wn=wn, name=name:
                           oracle.rmsnorm_residual(xn, rn, wn, 1e-6, dtype=name)]
            port_bytes += (rf.alg_bytes_rmsnorm(port_rows, h, dtype)
                           + rf.alg_bytes_rmsnorm_residual(port_rows, h, dtype))
    del pool
    rms = _rate(rms_bytes, _timed_passes(rms_cells, 0.5 * budget))
    del rms_cells

    # RoPE: q[4,2048,32,128] and k[4,2048,8,128], fp16 and bf16, tables cast
    # to the storage dtype.
    rope_cells, rope_bytes = [], 0
    cos32, sin32 = build_rope_tables(2048, 128)
    for dtype in (torch.float16, torch.bfloat16):
        cos, sin = cos32.to(dtype), sin32.to(dtype)
        q = torch.randn(4, 2048, 32, 128, generator=g).to(dtype)
        k = torch.randn(4, 2048, 8, 128, generator=g).to(dtype)
        rope_cells += [lambda q=q, c=cos, s=sin: rope_ref(q, c, s, "neox"),
                       lambda k=k, c=cos, s=sin: rope_ref(k, c, s, "neox")]
        rope_bytes += rf.alg_bytes_rope(4, 2048, 40, 128, dtype, dtype)
    rope = _rate(rope_bytes, _timed_passes(rope_cells, 0.2 * budget))
    del rope_cells

    gt = torch.randn(4096, 14336, generator=g).to(torch.bfloat16)
    ut = torch.randn(4096, 14336, generator=g).to(torch.bfloat16)
    swiglu = _rate(rf.alg_bytes_swiglu(4096, 14336, torch.bfloat16),
                   _timed_passes([lambda: swiglu_ref(gt, ut)], 0.15 * budget))
    del gt, ut

    port = _rate(port_bytes, _timed_passes(port_cells, 0.1 * budget))
    log(f"cpu baseline ({threads} threads): rmsnorm step {rms['value']} GB/s (passes {rms['spread']}), "
        f"rope q+k {rope['value']}, swiglu {swiglu['value']}; numpy oracle {port['value']} GB/s on 1 thread")
    return {
        **rms,
        "unit": "GB/s",
        "cores": threads,
        "os_cpu_count": os.cpu_count(),
        "kind": "port",
        "sample": (f"rmsnorm_ref/rmsnorm_residual_ref (ako/ops/rmsnorm_ref.py:8-50 restated) on host "
                   f"tensors: the step's 12 cells at full size ({RMS_ROWS} rows), median of passes"),
        "per_op": {
            "rope_qk": {**rope, "cells": "rope_ref q[4,2048,32,128]+k[4,2048,8,128], fp16 and bf16, full size"},
            "swiglu": {**swiglu, "cells": "swiglu_ref [4096,14336] bf16, full size"},
        },
        "gpu_speedup": round(value / rms["value"], 1) if rms["value"] > 0 else None,
        "oracle_numpy": {**port, "cores": 1, "cells": f"the same 12 cells with {port_rows} rows"},
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported. Split by rows or "
              "tokens (data or sequence parallelism), these kernels need no communication, so the "
              "N-GPU figure would be N times the one-GPU figure; it is not measured here.",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    from ako_amd import _native
    from ako_amd.benchmark import roofline as rf

    from ako_amd.benchmark.env import preflight, sample_env

    idle = preflight(0, strict=False)  # recorded next to the numbers, not enforced
    if idle["busy"]:
        log(f"warning: the GPU is not idle before timing: {idle}")
    _native.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    peak = rf.hbm_peak_gbps(dev)
    gen = torch.Generator(device=dev).manual_seed(0)

    def rnd(*shape, dtype, scale=1.0, shift=0.0):
        return (torch.randn(*shape, generator=gen, device=dev) * scale + shift).to(dtype)

    bytes_per_step, total_ms, per_launch = headline(args, torch, rf, dev, peak, rnd)
    ms_per_step = total_ms / args.steps
    value = bytes_per_step * args.steps / (total_ms * 1e-3) / 1e9
    log(f"timed: {ms_per_step:.3f} ms/step, {value:.1f} GB/s ({100 * value / peak:.1f}% of {peak:.0f})")
    dominant = max(per_launch, key=lambda s: s.mean_ms)
    ceilings = CopyCeilings(rf)
    b2b = headline_back_to_back(torch, rf, dev, rnd)
    per_kernel = []
    for stats in per_launch:
        row = stats.to_dict(peak)
        ceilings.annotate(row, stats.gbps())
        ms = b2b.get(stats.name)
        if ms:
            alone = rf.LaunchStats(stats.name, stats.alg_bytes, [ms])
            other = {"alg_bytes": stats.alg_bytes}
            ceilings.annotate(other, alone.gbps(), back_to_back=True)
            row["back_to_back"] = {"mean_us": round(ms * 1e3, 3), "pct_hbm_peak": round(100 * alone.gbps() / peak, 2),
                                   **{k: v for k, v in other.items() if k != "alg_bytes"}}
        per_kernel.append(row)

    roofline = {
        "bound": "hbm",
        "kernel": dominant.name,
        "achieved": round(dominant.gbps(), 1),
        "peak": peak,
        "unit": "GB/s",
        "frac": round(dominant.gbps() / peak, 4),
        "traffic": None,
        "alg_bytes_per_launch": dominant.alg_bytes,
        "mean_launch_us": round(dominant.mean_ms * 1e3, 2),
        "launches_timed": len(dominant.durations_ms),
        "timing": "HIP events bound to each launch (hipExtLaunchKernelGGL) on the launch stream, over K steps as value",
        # Which launches of this kernel (0-based, counted over the process) carry
        # the event pairs: after the warm-up passes, the K steps of `value` and
        # the lead passes. A kernel trace of the same run can be cut to exactly
        # these (python -m ako_amd.benchmark.rocprof --window).
        "event_launches": {"first": args.warmup + args.steps + rf.LEAD_PASSES, "count": args.steps},
    }
    if args.traffic.exists():
        from ako_amd.benchmark.rocprof import load_traffic_md

        measured = load_traffic_md(args.traffic)
        if dominant.name in measured:
            roofline["traffic"] = measured[dominant.name]
            roofline["traffic_source"] = str(args.traffic.relative_to(ROOT))
        for row in per_kernel:
            if row["name"] in measured:
                row["traffic_bytes"] = measured[row["name"]]
    copy = ceilings.get(dominant.alg_bytes)
    if copy is not None:
        roofline["copy_same_bytes"] = {
            "gbps": copy["gbps"],
            "frac": copy["frac"],
            "kernel_over_copy": round(dominant.gbps() / copy["gbps"], 4),
            "source": f"ako_amd/_lib/copy_ceiling {copy['bytes_per_buffer']}: 16-byte-packet copy, cold "
                      f"buffers, launch-bound events, {copy['block']}-lane groups, {copy.get('store', 'nt')} stores",
        }
        log(f"copy of the same bytes: {copy['gbps']:.0f} GB/s; the dominant kernel runs at "
            f"{100 * dominant.gbps() / copy['gbps']:.1f}% of it")

    extras, launch_floor, rope_prefill, decode_in_model = [], None, None, None
    if not args.no_extras:
        cells = extras_cells(torch, rf, dev, rnd)
        extras = time_extras(cells, torch, rf, peak, ceilings)
        del cells
        torch.cuda.empty_cache()
        rope_prefill = rope_prefill_summary(extras, ceilings)
        # The floor the graph_us figures sit on: a graph-replayed launch of a
        # kernel that does nothing measurable (torch's add_ on one element).
        tiny = torch.zeros(1, device=dev)
        launch_floor = {"graph_us": round(sorted(rf.time_graph_replay(lambda: tiny.add_(1.0)) for _ in range(5))[2], 3),
                        "kernel": "torch add_ on one element, 64 launches per graph, replayed"}
        log(f"extras: {len(extras)} cells timed; graph launch floor {launch_floor['graph_us']} us")
        decode_in_model = in_model_decode(torch, rf, dev, rnd)
        log("decode calls behind their producer GEMV (in model) / cold alone, us: " + ", ".join(
            f"{k} {v['graph_in_model_us']} / {v['graph_cold_us']}" for k, v in decode_in_model["ops"].items())
            + f"; {decode_in_model['step_library_us']} us per decode step")

    picked, comparisons = None, []
    if not args.no_selection:
        t0 = time.perf_counter()
        picked, comparisons = selection(torch)
        log(f"selection: HIP chosen in {picked['hip_selected']} of {picked['cells']} cells "
            f"({picked['decode_hip_selected']} of {picked['decode_cells']} decode cells) "
            f"in {time.perf_counter() - t0:.0f} s")

    decoder = None
    if not args.no_decoder:
        from ako_amd.models.bench_decoder import compare

        decoder = compare(prompt_len=512, decode_steps=128, repeats=3)
        log(f"decoder: prefill {decoder['torch']['prefill_ms']} -> {decoder['ako']['prefill_ms']} ms, "
            f"decode/step {decoder['torch']['decode_ms_per_step']} -> {decoder['ako']['decode_ms_per_step']} ms "
            f"(graphed {decoder['ako'].get('graphed_decode_ms_per_step')} ms)")
        torch.cuda.empty_cache()

    cpu = None if args.no_cpu else cpu_baseline(args, torch, rf, value)

    line = {
        "metric": "achieved HBM GB/s (% of peak) per op/shape; 4-layer decoder prefill+decode ms",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x, residual ~ N(0,1), weight ~ N(1, 0.1), seeded",
        "config": {
            "workload": "configs[1]: RMSNorm + residual RMSNorm, fp16 and bf16, 16384 rows x "
                        "hidden {4096, 8192, 16384}, eps 1e-6; one step = the 12 launches",
            "rows": RMS_ROWS,
            "hidden": list(RMS_HIDDEN),
            "storage_dtypes": ["fp16", "bf16"],
            "math": "fp32 (inputs widened, outputs rounded to nearest even)",
            "alg_bytes_per_step": bytes_per_step,
            "pct_hbm_peak": round(100 * value / peak, 2),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gpu_state": {"preflight": idle, "after": sample_env(0)},
        "selection": picked,
        "decoder": decoder,
        "rope_prefill": rope_prefill,
        "decode_in_model": decode_in_model,
        "per_kernel": per_kernel,
        "extras": extras,
        "launch_floor": launch_floor,
    }
    from ako_amd.benchmark.benchline import cells_report, compact_line, dumps_line
    from ako_amd.dispatcher.hardware import get_device_info

    info = get_device_info(dev)
    report = cells_report(line, info.to_dict(), info.device_name, comparisons)
    args.cells_out.parent.mkdir(parents=True, exist_ok=True)
    args.cells_out.write_text(json.dumps(report, indent=1))
    compact = compact_line(line)
    try:
        compact["cells_report"] = str(args.cells_out.resolve().relative_to(ROOT))
    except ValueError:
        compact["cells_report"] = str(args.cells_out)
    log(f"{len(report['results'])} cells and {len(comparisons)} selection rows written to {args.cells_out}")
    print(dumps_line(compact), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
