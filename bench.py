#!/usr/bin/env python
"""Headline benchmark: achieved HBM bandwidth of the HIP RMSNorm kernels.

One *step* is one pass of the hot path over the BASELINE.json configs[1]
prefill grid: plain RMSNorm and residual-add RMSNorm, fp16 and bf16, hidden
4096 / 8192 / 16384, 16384 rows (12 kernel launches, 11.27 GB of algorithmic
traffic). Inputs are resident in HBM before timing starts; consecutive
launches touch different buffers (11 GB per step against a 256 MB Infinity
Cache), so every launch reads cold data. ``value`` is algorithmic bytes per
step x steps / elapsed device time, in GB/s.

Also reported on the same line:
  roofline      the dominant kernel (largest share of the step) with its
                per-launch duration from HIP events on the launch stream,
                and a plain device copy of the same byte count timed the same
                way (copy_same_bytes: the size's practical ceiling);
  per_kernel    every launch of the step;
  extras        the RoPE and SwiGLU cells, the
                decode-size RMSNorm cells, the KV-cache RoPE and the
                tensor-parallel RMSNorm halves;
  decoder       configs[4]: the 4-layer fp16 decoder, prefill 512 tokens then
                128 greedy steps, eager PyTorch vs the dispatcher, each also
                with decode steps replayed from a HIP graph;
  cpu_baseline  the oracle (numpy port of the reference's unfused path, one
                thread) on the same grid with a bounded row sample, and beside
                it the restated PyTorch reference on host CPU tensors.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

RMS_HIDDEN = (4096, 8192, 16384)
RMS_ROWS = 16384


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-extras", action="store_true", help="skip the RoPE/SwiGLU/decode cells")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decoder", action="store_true", help="skip the configs[4] decoder run")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--traffic", type=Path, default=ROOT / "profiles" / "hbm_traffic_hot_path_cells.md",
                    help="rocprofv3 FETCH/WRITE summary (ako_amd.benchmark.rocprof) for the kernels")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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
    from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
    from ako_amd.ops.rope_hip import rope_hip, rope_qk_cache_hip, rope_qk_hip
    from ako_amd.ops.rope_ref import build_rope_tables
    from ako_amd.ops.swiglu_hip import swiglu_hip

    _native.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    peak = rf.hbm_peak_gbps(dev)
    gen = torch.Generator(device=dev).manual_seed(0)

    def rnd(*shape, dtype, scale=1.0, shift=0.0):
        return (torch.randn(*shape, generator=gen, device=dev) * scale + shift).to(dtype)

    # ---- the metric's workload: configs[1] prefill grid ------------------------
    calls = []
    for dtype in (torch.float16, torch.bfloat16):
        tag = "fp16" if dtype == torch.float16 else "bf16"
        for h in RMS_HIDDEN:
            x = rnd(RMS_ROWS, h, dtype=dtype)
            r = rnd(RMS_ROWS, h, dtype=dtype)
            w = rnd(h, dtype=dtype, scale=0.1, shift=1.0)
            calls.append((f"rmsnorm_{tag}_{RMS_ROWS}x{h}", rf.alg_bytes_rmsnorm(RMS_ROWS, h, dtype),
                          lambda x=x, w=w: rmsnorm_hip(x, w, 1e-6)))
            calls.append((f"rmsnorm_residual_{tag}_{RMS_ROWS}x{h}",
                          rf.alg_bytes_rmsnorm_residual(RMS_ROWS, h, dtype),
                          lambda x=x, r=r, w=w: rmsnorm_residual_hip(x, r, w, 1e-6)))
    bytes_per_step = sum(b for _, b, _ in calls)
    log(f"workload: {len(calls)} launches/step, {bytes_per_step / 1e9:.3f} GB/step, "
        f"warmup {args.warmup}, steps {args.steps}")
    rf.warm(calls, args.warmup)
    total_ms = rf.time_steps(calls, steps=args.steps)
    ms_per_step = total_ms / args.steps
    value = bytes_per_step * args.steps / (total_ms * 1e-3) / 1e9
    log(f"timed: {ms_per_step:.3f} ms/step, {value:.1f} GB/s ({100 * value / peak:.1f}% of {peak:.0f})")
    # The dominant kernel's launch duration: the same K steps again, now with an
    # event pair around every launch (kept out of the region above so that the
    # step time holds nothing but the kernels and their launches).
    per_launch = rf.time_each_launch(calls, steps=args.steps)
    dominant = max(per_launch, key=lambda s: s.mean_ms)
    per_kernel = [s.to_dict(peak) for s in per_launch]

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
        "timing": "HIP events around each launch on the launch stream, over the same K steps as value",
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
    copy = rf.copy_same_bytes(dominant.alg_bytes)
    if copy is not None:
        roofline["copy_same_bytes"] = {
            "gbps": copy["gbps"],
            "frac": copy["frac"],
            "kernel_over_copy": round(dominant.gbps() / copy["gbps"], 4),
            "source": f"ako_amd/_lib/copy_ceiling {copy['bytes_per_buffer']} (plain 16-byte-packet copy "
                      f"moving {copy['traffic_bytes']} bytes, cold buffers, per-launch events, "
                      f"{copy['block']}-lane workgroups, {copy.get('store', 'nt')} stores; the fastest copy found)",
        }
        log(f"copy of the same bytes: {copy['gbps']:.0f} GB/s; the dominant kernel runs at "
            f"{100 * dominant.gbps() / copy['gbps']:.1f}% of it")
    del calls
    torch.cuda.empty_cache()

    # ---- other configs' cells (reported, not the metric) ----------------------
    extras = []
    launch_floor = None
    if not args.no_extras:
        cells = []
        for dtype in (torch.float16, torch.bfloat16):
            tag = "fp16" if dtype == torch.float16 else "bf16"
            for b, s in ((4, 2048), (64, 1), (1, 1)):
                cos, sin = build_rope_tables(s, 128, device=dev)
                cos, sin = cos.to(dtype), sin.to(dtype)
                copies = rf.copies_for_cold(rf.alg_bytes_rope(b, s, 40, 128, dtype, dtype), dev) if s > 1 else 1
                qs = [rnd(b, s, 32, 128, dtype=dtype) for _ in range(copies)]
                ks = [rnd(b, s, 8, 128, dtype=dtype) for _ in range(copies)]
                for i in range(copies):
                    cells.append((f"rope_q_{tag}_{b}x{s}x32x128", rf.alg_bytes_rope(b, s, 32, 128, dtype, dtype),
                                  lambda q=qs[i], c=cos, sn=sin: rope_hip(q, c, sn, "neox")))
                    cells.append((f"rope_k_{tag}_{b}x{s}x8x128", rf.alg_bytes_rope(b, s, 8, 128, dtype, dtype),
                                  lambda k=ks[i], c=cos, sn=sin: rope_hip(k, c, sn, "neox")))
                    cells.append((f"rope_qk_{tag}_{b}x{s}", rf.alg_bytes_rope(b, s, 40, 128, dtype, dtype),
                                  lambda q=qs[i], k=ks[i], c=cos, sn=sin: rope_qk_hip(q, k, c, sn, "neox")))
        # configs[4] decode step, one layer: RoPE of q and k plus the KV-cache
        # append, fused (one launch) and as the unfused sequence it replaces.
        dtype = torch.float16
        full_cos, full_sin = build_rope_tables(640, 128, device=dev)
        q1, k1, v1 = rnd(1, 1, 32, 128, dtype=dtype), rnd(1, 1, 32, 128, dtype=dtype), rnd(1, 1, 32, 128, dtype=dtype)
        kc, vc = rnd(1, 32, 640, 128, dtype=dtype), rnd(1, 32, 640, 128, dtype=dtype)
        pos = torch.full((1,), 511, dtype=torch.long, device=dev)
        cache_bytes = rf.alg_bytes_rope_qk_cache(1, 1, 32, 32, 128, dtype, torch.float32)

        def unfused_cache_step():
            c, sn = full_cos.index_select(0, pos), full_sin.index_select(0, pos)
            qo, ko = rope_qk_hip(q1, k1, c, sn, "neox")
            kc.index_copy_(2, pos, ko.transpose(1, 2))
            vc.index_copy_(2, pos, v1.transpose(1, 2))
            return qo

        cells.append(("rope_qk_cache_fp16_1x1_q32_kv32_slot511of640", cache_bytes,
                      lambda: rope_qk_cache_hip(q1, k1, v1, full_cos, full_sin, pos, kc, vc, "neox")))
        cells.append(("rope_qk_then_index_copy_fp16_1x1_q32_kv32", cache_bytes, unfused_cache_step))
        # One tensor-parallel rank's slice of the widest configs[1] row (TP=8:
        # 2048 of 16384): residual + partial sum of squares, then the apply half.
        from ako_amd.ops.rmsnorm_tp import rmsnorm_shard_apply_hip, rmsnorm_shard_partial_hip

        for dtype in (torch.float16, torch.bfloat16):
            tag = "fp16" if dtype == torch.float16 else "bf16"
            rows_tp, shard = RMS_ROWS, 2048
            nb_p = rf.alg_bytes_rmsnorm_shard_partial(rows_tp, shard, dtype, residual=True)
            nb_a = rf.alg_bytes_rmsnorm_shard_apply(rows_tp, shard, dtype)
            copies = rf.copies_for_cold(nb_p, dev)
            xs_tp = [rnd(rows_tp, shard, dtype=dtype) for _ in range(copies)]
            rs_tp = [rnd(rows_tp, shard, dtype=dtype) for _ in range(copies)]
            w_tp = rnd(shard, dtype=dtype, scale=0.1, shift=1.0)
            tot = torch.full((rows_tp,), float(shard), device=dev)
            for i in range(copies):
                cells.append((f"rmsnorm_shard_partial_{tag}_{rows_tp}x{shard}_residual", nb_p,
                              lambda x=xs_tp[i], r=rs_tp[i]: rmsnorm_shard_partial_hip(x, r)))
                cells.append((f"rmsnorm_shard_apply_{tag}_{rows_tp}x{shard}", nb_a,
                              lambda s_=xs_tp[i], w_=w_tp, t_=tot: rmsnorm_shard_apply_hip(s_, w_, t_, 8 * shard, 1e-6)))
        for m in (16384, 4096, 256, 16, 1):
            dtype = torch.bfloat16
            nbytes = rf.alg_bytes_swiglu(m, 14336, dtype)
            copies = rf.copies_for_cold(nbytes, dev) if m >= 256 else 1
            gs = [rnd(m, 14336, dtype=dtype) for _ in range(copies)]
            us = [rnd(m, 14336, dtype=dtype) for _ in range(copies)]
            for i in range(copies):
                cells.append((f"swiglu_bf16_{m}x14336", nbytes, lambda g=gs[i], u=us[i]: swiglu_hip(g, u)))
        for dtype in (torch.float16, torch.bfloat16):
            tag = "fp16" if dtype == torch.float16 else "bf16"
            for rows in (1, 32):
                for h in RMS_HIDDEN:
                    x, r = rnd(rows, h, dtype=dtype), rnd(rows, h, dtype=dtype)
                    w = rnd(h, dtype=dtype, scale=0.1, shift=1.0)
                    cells.append((f"rmsnorm_{tag}_{rows}x{h}", rf.alg_bytes_rmsnorm(rows, h, dtype),
                                  lambda x=x, w=w: rmsnorm_hip(x, w, 1e-6)))
                    cells.append((f"rmsnorm_residual_{tag}_{rows}x{h}",
                                  rf.alg_bytes_rmsnorm_residual(rows, h, dtype),
                                  lambda x=x, r=r, w=w: rmsnorm_residual_hip(x, r, w, 1e-6)))
        rf.warm(cells, 2)
        # Each cell: 60 back-to-back launches over its input copies between one
        # event pair (per-launch events would distort 5-30 us kernels), and for
        # decode-size cells the device time per call from a replayed HIP graph
        # of 64 launches (no host overhead), the median of five such timings.
        groups: dict[str, list] = {}
        for name, nbytes, fn in cells:
            groups.setdefault(name, [nbytes, []])[1].append(fn)
        for name, (nbytes, fns) in groups.items():
            ms = rf.time_back_to_back(fns, launches=60)
            stats = rf.LaunchStats(name, nbytes, [ms])
            row = stats.to_dict(peak)
            row.pop("launches")
            row.pop("p50_us")
            row["copies"] = len(fns)
            if nbytes < 64 * 2**20:
                # Median of five graph timings: one is under a millisecond of
                # device time, and clock changes move single readings by up to 15%.
                row["graph_us"] = round(sorted(rf.time_graph_replay(fns[0]) for _ in range(5))[2], 3)
            extras.append(row)
        # The floor those graph_us figures sit on: a graph-replayed launch of a
        # kernel that does nothing measurable (torch's add_ on one element).
        tiny = torch.zeros(1, device=dev)
        launch_floor = {"graph_us": round(sorted(rf.time_graph_replay(lambda: tiny.add_(1.0)) for _ in range(5))[2], 3),
                        "kernel": "torch add_ on one element, 64 launches per graph, replayed"}
        log(f"extras: {len(extras)} cells timed; graph launch floor {launch_floor['graph_us']} us")
        del cells
        torch.cuda.empty_cache()

    # ---- the 4-layer decoder, prefill 512 + 128 greedy steps -------
    decoder = None
    if not args.no_decoder:
        from ako_amd.models.bench_decoder import compare

        decoder = compare(prompt_len=512, decode_steps=128, repeats=3)
        log(f"decoder: prefill {decoder['torch']['prefill_ms']} -> {decoder['ako']['prefill_ms']} ms, "
            f"decode/step {decoder['torch']['decode_ms_per_step']} -> {decoder['ako']['decode_ms_per_step']} ms "
            f"(graphed {decoder['ako'].get('graphed_decode_ms_per_step')} ms)")
        torch.cuda.empty_cache()

    # ---- CPU baseline: the oracle (a CPU port of the reference's algorithm) ------
    # The oracle (numpy, single-threaded) is the primary figure, as a "port" of
    # the reference's unfused path; the restated PyTorch reference on host
    # tensors (multi-threaded) is reported beside it. Both run the 12 cells of
    # the step on a bounded row sample, timed by wall clock for ~cpu-seconds.
    cpu = None
    if not args.no_cpu:
        import numpy as np

        from ako_amd.ops.rmsnorm_ref import rmsnorm_ref, rmsnorm_residual_ref
        from oracle import ops as oracle

        def storage(t: "torch.Tensor") -> "np.ndarray":
            if t.dtype == torch.bfloat16:
                return t.view(torch.int16).numpy().view(np.uint16)
            return t.numpy()

        def timed_passes(cells: list, seconds: float) -> tuple[int, float]:
            for _, fn in cells:
                fn()
            passes, t0 = 0, time.perf_counter()
            while True:
                for _, fn in cells:
                    fn()
                passes += 1
                elapsed = time.perf_counter() - t0
                if elapsed >= seconds and passes >= 3:
                    return passes, elapsed

        sample_rows = 64
        g = torch.Generator().manual_seed(0)
        port_cells, torch_cells = [], []
        for dtype in (torch.float16, torch.bfloat16):
            name = "float16" if dtype == torch.float16 else "bfloat16"
            for h in RMS_HIDDEN:
                x = torch.randn(sample_rows, h, generator=g).to(dtype)
                r = torch.randn(sample_rows, h, generator=g).to(dtype)
                w = (torch.randn(h, generator=g) * 0.1 + 1.0).to(dtype)
                xn, rn, wn = storage(x), storage(r), storage(w)
                b_plain = rf.alg_bytes_rmsnorm(sample_rows, h, dtype)
                b_res = rf.alg_bytes_rmsnorm_residual(sample_rows, h, dtype)
                port_cells.append((b_plain, lambda xn=xn, wn=wn, name=name: oracle.rmsnorm(xn, wn, 1e-6, dtype=name)))
                port_cells.append((b_res, lambda xn=xn, rn=rn, wn=wn, name=name:
                                   oracle.rmsnorm_residual(xn, rn, wn, 1e-6, dtype=name)))
                torch_cells.append((b_plain, lambda x=x, w=w: rmsnorm_ref(x, w, 1e-6)))
                torch_cells.append((b_res, lambda x=x, r=r, w=w: rmsnorm_residual_ref(x, r, w, 1e-6)))
        passes, elapsed = timed_passes(port_cells, args.cpu_seconds)
        port_gbps = sum(b for b, _ in port_cells) * passes / elapsed / 1e9
        t_passes, t_elapsed = timed_passes(torch_cells, args.cpu_seconds / 2)
        torch_gbps = sum(b for b, _ in torch_cells) * t_passes / t_elapsed / 1e9
        cpu = {
            "value": round(port_gbps, 3),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": (f"oracle.ops.rmsnorm / rmsnorm_residual (numpy restatement of the reference's "
                       f"unfused path, one thread) on the same 12 cells with {sample_rows} rows instead "
                       f"of {RMS_ROWS}: {passes} passes in {elapsed:.1f} s"),
            "gpu_speedup": round(value / port_gbps, 1) if port_gbps > 0 else None,
            "torch_cpu": {
                "value": round(torch_gbps, 3),
                "cores": torch.get_num_threads(),
                "sample": (f"ako_amd.ops.rmsnorm_ref / rmsnorm_residual_ref (the reference's PyTorch "
                           f"path) on host tensors, same cells: {t_passes} passes in {t_elapsed:.1f} s; "
                           f"os.cpu_count()={os.cpu_count()}"),
            },
        }
        log(f"cpu baseline: oracle {port_gbps:.3f} GB/s on 1 thread, torch CPU {torch_gbps:.3f} GB/s "
            f"on {torch.get_num_threads()} threads")

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
        "decoder": decoder,
        "per_kernel": per_kernel,
        "extras": extras,
        "launch_floor": launch_floor,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
