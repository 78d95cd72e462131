"""Offline selection for one inference workload, written as a runtime config.

The reference's ``scripts/optimize_model.py:31-151`` runs the selection
(gate, timing, cache record) once for every operation on the shapes a decoder
layer of the workload uses, and writes ``selected_config.json`` so that a
serving process starts with its decisions made. Here the operations are the
four of this library plus the fused ``rope_qk`` (q and k in one launch, the
way the decoder calls RoPE), and a workload can be given either by its
dimensions or as ``--preset config5``: the BASELINE.json configs[4] decoder at
prefill (512 tokens) and at a decode step (1 token), both selected.

    python -m ako_amd.benchmark.optimize --output-dir reports/mi355x [--preset config5]
        [--batch-size 8 --seq-len 2048 --hidden-dim 4096 --num-heads 32 --head-dim 128
         --ffn-dim 11008 --dtype fp16]

The document layout is the reference's (``gpu``, ``compute_backend``,
``device``, ``created_at``, ``parameters``, ``operations``, ``cache``); with a
preset, ``operations`` holds one entry per phase (``prefill/rmsnorm``, ...).
"""

from __future__ import annotations

import argparse
import json
import sys
from dataclasses import dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import torch

from ako_amd.benchmark.bench_op import parse_dtypes
from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.hardware import get_device_info
from ako_amd.dispatcher.registry import KernelRegistry
from ako_amd.dispatcher.selector import KernelSelector, SelectionResult
from ako_amd.ops._registry import register_all
from ako_amd.ops.rope_ref import build_rope_tables


@dataclass
class Workload:
    """The shapes one decoder layer of a workload feeds the four operations."""

    batch_size: int = 8
    seq_len: int = 2048
    hidden_dim: int = 4096
    num_heads: int = 32
    num_kv_heads: int = 32
    head_dim: int = 128
    ffn_dim: int = 11008
    dtype: torch.dtype = torch.float16
    rope_style: str = "neox"

    def tensors(self, device: torch.device, seed: int = 0) -> dict[str, tuple[tuple[torch.Tensor, ...], dict[str, Any]]]:
        """Seeded inputs per operation: ``{op: (tensors, call_kwargs)}``."""
        g = torch.Generator(device="cpu").manual_seed(seed)

        def rnd(*shape, scale=1.0, shift=0.0):
            return (torch.randn(*shape, generator=g) * scale + shift).to(device=device, dtype=self.dtype)

        b, s = self.batch_size, self.seq_len
        hidden = rnd(b, s, self.hidden_dim)
        weight = rnd(self.hidden_dim, scale=0.1, shift=1.0)
        q = rnd(b, s, self.num_heads, self.head_dim)
        k = rnd(b, s, self.num_kv_heads, self.head_dim)
        cos, sin = build_rope_tables(s, self.head_dim, device=device, dtype=torch.float32)
        style = {"style": self.rope_style}
        return {
            "rmsnorm": ((hidden, weight), {}),
            "rmsnorm_residual": ((hidden, rnd(b, s, self.hidden_dim), weight), {}),
            "rope": ((q, cos, sin), style),
            "rope_qk": ((q, k, cos, sin), style),
            "swiglu": ((rnd(b, s, self.ffn_dim), rnd(b, s, self.ffn_dim)), {}),
        }

    def parameters(self) -> dict[str, Any]:
        return {"batch_size": self.batch_size, "seq_len": self.seq_len, "hidden_dim": self.hidden_dim,
                "num_heads": self.num_heads, "num_kv_heads": self.num_kv_heads, "head_dim": self.head_dim,
                "ffn_dim": self.ffn_dim, "dtype": str(self.dtype).removeprefix("torch."),
                "rope_style": self.rope_style}


def config5_phases() -> dict[str, Workload]:
    """hidden 4096, 32 x 128 heads (MHA), FFN 11008,
    fp16, batch 1; a 512-token prefill and a one-token decode step."""
    common = dict(batch_size=1, hidden_dim=4096, num_heads=32, num_kv_heads=32, head_dim=128, ffn_dim=11008,
                  dtype=torch.float16)
    return {"prefill": Workload(seq_len=512, **common), "decode": Workload(seq_len=1, **common)}


def select_workload(selector: KernelSelector, workload: Workload, device: torch.device) -> list[SelectionResult]:
    out = []
    for op, (tensors, kwargs) in workload.tensors(device).items():
        out.append(selector.select_entry(op, *tensors, extra_key=kwargs.get("style"), call_kwargs=kwargs))
    return out


def optimize(phases: dict[str, Workload], *, device: torch.device, cache: KernelCache, warmup: int = 10,
             repeats: int = 30, allow_cpu_tuning: bool = False) -> dict[str, Any]:
    """Run the selection for every phase and return the config document."""
    info = get_device_info(device)
    selector = KernelSelector(registry=register_all(KernelRegistry()), cache=cache, auto_tune=True,
                              allow_cpu_tuning=allow_cpu_tuning, warmup=warmup, repeats=repeats)
    operations: dict[str, Any] = {}
    for phase, workload in phases.items():
        for sel in select_workload(selector, workload, device):
            key = sel.op_name if len(phases) == 1 else f"{phase}/{sel.op_name}"
            operations[key] = sel.to_dict()
    params = ({name: w.parameters() for name, w in phases.items()} if len(phases) > 1
              else next(iter(phases.values())).parameters())
    return {
        "gpu": info.device_name,
        "compute_backend": info.compute_backend,
        "device": info.to_dict(),
        "created_at": datetime.now(timezone.utc).isoformat(),
        "parameters": params,
        "operations": operations,
        "cache": {"path": str(cache.path), **cache.stats().to_dict()},
    }


def summary_lines(config: dict[str, Any]) -> list[str]:
    lines = []
    for name, op in config["operations"].items():
        lat = op.get("latency_p50_ms")
        vs = op.get("speedup_vs_best_baseline")
        lines.append(f"{name:26s} {op.get('selected_kernel', '?'):24s} {op.get('backend', '?'):8s} "
                     f"{(f'{lat * 1e3:.1f} us' if lat else '-'):>10s} "
                     f"{(f'{vs:.2f}x vs best baseline' if vs else ''):>24s} [{op.get('source', '?')}]")
    return lines


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--output-dir", type=Path, default=Path("reports"))
    ap.add_argument("--device", default="cuda" if torch.cuda.is_available() else "cpu")
    ap.add_argument("--preset", choices=("config5",), default=None)
    ap.add_argument("--batch-size", type=int, default=8)
    ap.add_argument("--seq-len", type=int, default=2048)
    ap.add_argument("--hidden-dim", type=int, default=4096)
    ap.add_argument("--num-heads", type=int, default=32)
    ap.add_argument("--num-kv-heads", type=int, default=None)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--ffn-dim", type=int, default=11008)
    ap.add_argument("--dtype", default="fp16", choices=("fp16", "bf16", "fp32"))
    ap.add_argument("--rope-style", default="neox", choices=("neox", "interleaved"))
    ap.add_argument("--cache-path", type=Path, default=None)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--repeats", type=int, default=30)
    ap.add_argument("--allow-cpu-tuning", action="store_true",
                    help="time candidates on the CPU too (off by default: only the baselines run there)")
    ap.add_argument("--fresh", action="store_true", help="ignore and overwrite cached decisions")
    args = ap.parse_args(argv)

    device = torch.device(args.device)
    if args.preset == "config5":
        phases = config5_phases()
    else:
        (dtype,) = parse_dtypes([args.dtype])
        phases = {"workload": Workload(args.batch_size, args.seq_len, args.hidden_dim, args.num_heads,
                                       args.num_kv_heads or args.num_heads, args.head_dim, args.ffn_dim,
                                       dtype, args.rope_style)}
    cache = KernelCache(path=args.cache_path)
    if args.fresh:
        cache.clear()
    config = optimize(phases, device=device, cache=cache, warmup=args.warmup, repeats=args.repeats,
                      allow_cpu_tuning=args.allow_cpu_tuning)
    print("\n".join(summary_lines(config)), flush=True)
    args.output_dir.mkdir(parents=True, exist_ok=True)
    path = args.output_dir / "selected_config.json"
    path.write_text(json.dumps(config, indent=2))
    print(f"selected config written to {path}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
