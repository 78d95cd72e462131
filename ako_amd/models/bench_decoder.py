"""4-layer decoder, prefill 512 tokens + 128 greedy steps.

fp16, random init N(0, 0.02), hidden 4096, 32 heads x 128, FFN 11008, RMSNorm
eps 1e-6, RoPE theta 1e4, batch 1. GEMMs and attention run on PyTorch-ROCm;
RMSNorm / residual RMSNorm / RoPE / SwiGLU go through the ``ako_amd``
dispatcher (``backend="ako"``) or the unfused eager references
(``backend="torch"``). Reported per backend: prefill ms, decode ms (all 128
steps and per step), wall clock around a synchronised region, plus the
generated tokens so the two backends can be compared. Prefill is the median of
20 passes after 3 untimed ones; decode the median of 3 full 128-step runs. Each backend is also
run with every decode step replayed from a HIP graph (``GraphedGreedy``),
which removes the per-launch host cost that dominates batch-1 decoding.

    python -m ako_amd.models.bench_decoder [--steps 128] [--prompt 512] [--backend ako]
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from typing import Any

import torch

from ako_amd.models.decoder import GraphedGreedy, build_lm, config5


def _timed(fn) -> tuple[Any, float]:
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = fn()
    torch.cuda.synchronize()
    return out, (time.perf_counter() - t0) * 1e3


def _fold(rows: list[dict[str, Any]], share: dict[str, Any], per: int) -> dict[str, Any]:
    return {
        "device_us": round(share["total_us"] / per, 1),
        "library_us": round(share["library_us"] / per, 1),
        "library_share": round(share["share"], 4),
        "library_launches": round(share["library_calls"] / per, 2),
        "library_kernels": share["library_kernels"],
        "top": [{"name": r["name"][:80], "us": round(r["total_us"] / per, 2),
                 "calls": round(r["calls"] / per, 2)} for r in rows[:8]],
    }


def prefill_breakdown(model, prompt: torch.Tensor, passes: int = 5) -> dict[str, Any]:
    """Where a prefill pass's device time goes (``passes`` prefills into fresh
    caches under ``torch.profiler``, folded by kernel name, per pass), with
    the share of this library's kernels."""
    from ako_amd.benchmark.profiler import kernel_table, library_share, profile_cuda

    caches = [model.stack.new_kv_cache(prompt.shape[1] + 1) for _ in range(passes)]
    model.logits_last(prompt, model.stack.new_kv_cache(prompt.shape[1] + 1))  # warm
    torch.cuda.synchronize()
    with profile_cuda() as prof:
        for cache in caches:
            model.logits_last(prompt, cache)
        torch.cuda.synchronize()
    rows = kernel_table(prof, device=True)
    share = library_share(rows)
    if not rows or share["total_us"] <= 0:
        return {"passes": passes, "recorded": False}
    return {"passes": passes, "recorded": True, **_fold(rows, share, passes)}


def graphed_step_breakdown(model, prompt: torch.Tensor, steps: int = 32) -> dict[str, Any]:
    """Where a graph-replayed decode step's device time goes: ``steps`` replays
    recorded with ``torch.profiler`` and folded by kernel name, with the share
    of this library's kernels (``ako::``). Profiling adds a little time per
    kernel, so the totals here run above the untraced step time."""
    from ako_amd.benchmark.profiler import kernel_table, library_share, profile_cuda

    runner = GraphedGreedy(model, prompt, steps + 1)
    torch.cuda.synchronize()
    with profile_cuda() as prof:
        runner.run()
        torch.cuda.synchronize()
    rows = kernel_table(prof, device=True)
    share = library_share(rows)
    del runner
    if not rows or share["total_us"] <= 0:
        return {"steps": steps, "recorded": False}
    return {
        "steps": steps,
        "recorded": True,
        "device_us_per_step": round(share["total_us"] / steps, 1),
        "library_us_per_step": round(share["library_us"] / steps, 1),
        "library_share": round(share["share"], 4),
        "library_launches_per_step": round(share["library_calls"] / steps, 2),
        "library_kernels": share["library_kernels"],
        "top": [{"name": r["name"][:80], "us_per_step": round(r["total_us"] / steps, 2),
                 "calls_per_step": round(r["calls"] / steps, 2)} for r in rows[:8]],
    }


def run_config5(backend: str, *, prompt_len: int = 512, decode_steps: int = 128, repeats: int = 3,
                device: str = "cuda", seed: int = 0, graphed: bool = True, prefill_warmup: int = 3,
                prefill_repeats: int = 20, breakdown: bool = False, fused_qkv: bool = True) -> dict[str, Any]:
    cfg = config5()
    cfg.max_seq_len = prompt_len + decode_steps
    cfg.fused_qkv = fused_qkv
    model = build_lm(cfg, backend=backend, device=device, dtype=torch.float16, seed=seed)
    gen = torch.Generator(device="cpu").manual_seed(seed)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=gen).to(device)

    with torch.no_grad():
        model.generate_greedy(prompt, decode_steps)  # warmup, incl. first-sight kernel selection
        # Prefill on its own: a few untimed passes, then the median of many
        # (one pass is ~2 ms, so a handful of samples is at the mercy of clock
        # ramp-up after the host-bound decode loop).
        prefill_ms = []
        for i in range(prefill_warmup + prefill_repeats):
            cache = model.stack.new_kv_cache(prompt_len + decode_steps)
            _, t_pre = _timed(lambda: model.logits_last(prompt, cache).argmax(-1, keepdim=True))
            if i >= prefill_warmup:
                prefill_ms.append(t_pre)
        decode_ms, tokens = [], None
        for _ in range(repeats):
            cache = model.stack.new_kv_cache(prompt_len + decode_steps)
            nxt = model.logits_last(prompt, cache).argmax(-1, keepdim=True)

            def decode(nxt=nxt, cache=cache):
                out = [nxt]
                for _ in range(decode_steps - 1):
                    nxt = model.logits_last(nxt, cache).argmax(-1, keepdim=True)
                    out.append(nxt)
                return torch.cat(out, dim=1)

            tokens, t_dec = _timed(decode)
            decode_ms.append(t_dec)
        graphed_ms, graphed_tokens = [], None
        if graphed:
            for _ in range(repeats):
                runner = GraphedGreedy(model, prompt, decode_steps)
                graphed_tokens, t_g = _timed(runner.run)
                graphed_ms.append(t_g)
                del runner
        step_breakdown = graphed_step_breakdown(model, prompt) if (graphed and breakdown) else None
        prefill_parts = prefill_breakdown(model, prompt) if breakdown else None
    prefill = sorted(prefill_ms)[len(prefill_ms) // 2]
    dec = sorted(decode_ms)[len(decode_ms) // 2]
    extra = {}
    if graphed_ms:
        g = sorted(graphed_ms)[len(graphed_ms) // 2]
        extra = {
            "graphed_decode_ms": round(g, 3),
            "graphed_decode_ms_per_step": round(g / max(decode_steps - 1, 1), 4),
            "graphed_tokens_match_eager": bool(torch.equal(graphed_tokens.cpu(), tokens.cpu())),
        }
    return {
        "backend": backend,
        "prefill_ms": round(prefill, 3),
        "prefill_samples": len(prefill_ms),
        "decode_ms": round(dec, 3),
        "decode_ms_per_step": round(dec / max(decode_steps - 1, 1), 4),
        "prompt_len": prompt_len,
        "decode_steps": decode_steps,
        "tokens": tokens[0].tolist(),
        **extra,
        **({"graphed_step_breakdown": step_breakdown} if step_breakdown is not None else {}),
        **({"prefill_breakdown": prefill_parts} if prefill_parts is not None else {}),
    }


def compare(prompt_len: int = 512, decode_steps: int = 128, repeats: int = 3,
            fused_qkv: bool = True) -> dict[str, Any]:
    """Both backends on the same weights and the same projection layout: the
    difference between them is the four operations' kernels alone."""
    results = {b: run_config5(b, prompt_len=prompt_len, decode_steps=decode_steps, repeats=repeats,
                              breakdown=(b == "ako"), fused_qkv=fused_qkv)
               for b in ("torch", "ako")}
    ta, tt = results["ako"]["tokens"], results["torch"]["tokens"]
    first_diff = next((i for i, (a, b) in enumerate(zip(ta, tt)) if a != b), None)
    for r in results.values():
        r.pop("tokens")
    return {
        "config": "configs[4]: 4 layers, hidden 4096, 32x128 heads, FFN 11008, fp16, vocab 32000, MHA",
        "qkv_projection": "fused" if fused_qkv else "separate",
        "torch": results["torch"],
        "ako": results["ako"],
        "prefill_speedup": round(results["torch"]["prefill_ms"] / results["ako"]["prefill_ms"], 3),
        "decode_speedup": round(results["torch"]["decode_ms"] / results["ako"]["decode_ms"], 3),
        "graphed_decode_speedup": (
            round(results["torch"]["graphed_decode_ms"] / results["ako"]["graphed_decode_ms"], 3)
            if "graphed_decode_ms" in results["ako"] else None),
        "greedy_tokens_identical": first_diff is None,
        "first_token_mismatch": first_diff,
    }


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--backend", choices=("torch", "ako"), default=None,
                    help="run one backend only (e.g. under a profiler) instead of comparing both")
    ap.add_argument("--separate-qkv", action="store_true",
                    help="three q/k/v projections (the reference's layout) instead of one fused GEMM")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("configs[4] needs a GPU", file=sys.stderr)
        return 1
    if args.backend:
        out = run_config5(args.backend, prompt_len=args.prompt, decode_steps=args.steps, repeats=args.repeats,
                          fused_qkv=not args.separate_qkv)
        out.pop("tokens")
    else:
        out = compare(args.prompt, args.steps, args.repeats, fused_qkv=not args.separate_qkv)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
