"""Writes the committed fixtures of this directory. Run from the repo root:

    python tests/golden/make_golden.py

known_answers.json  closed forms evaluated in float64 with the ``math``
                    module only (independent of numpy and torch): RMSNorm of
                    [[3, 4]], RoPE tables and rotations at small positions,
                    SiLU at fixed points.
reference_golden.json  values the reference repository itself records for
                    this path, read as data from /root/reference (which
                    exists only in the build container): the rejection line
                    printed in docs/EXTENDING.md, the cache keys of
                    reports/rtx3070/selected_config_{fp16,bf16}.json, and
                    the ulp known answers of tests/test_tolerance.py:21-27.
"""

from __future__ import annotations

import json
import math
import re
from pathlib import Path

HERE = Path(__file__).resolve().parent
REFERENCE = Path("/root/reference")


def rope_tables64(seq: int, head_dim: int, base: float = 10000.0, offset: int = 0):
    half = head_dim // 2
    inv = [1.0 / base ** (2.0 * i / head_dim) for i in range(half)]
    ang = [[(offset + p) * f for f in inv] for p in range(seq)]
    return [[math.cos(a) for a in row] for row in ang], [[math.sin(a) for a in row] for row in ang]


def rotate64(vec: list[float], cos_row: list[float], sin_row: list[float], style: str) -> list[float]:
    d = len(vec)
    half = d // 2
    out = [0.0] * d
    for i in range(half):
        ia, ib = (i, i + half) if style == "neox" else (2 * i, 2 * i + 1)
        a, b, c, s = vec[ia], vec[ib], cos_row[i], sin_row[i]
        out[ia] = a * c - b * s
        out[ib] = a * s + b * c
    return out


def known_answers() -> dict:
    eps = 1e-6
    rms = math.sqrt((9.0 + 16.0) / 2.0 + eps)
    cos, sin = rope_tables64(4, 8)
    vec = [1.0, -2.0, 3.0, -4.0, 0.5, 0.25, -1.5, 2.0]
    silu_points = [-20.0, -5.0, -1.0, -0.5, 0.0, 0.5, 1.0, 5.0, 20.0]
    return {
        "rmsnorm_3_4": {"x": [[3.0, 4.0]], "w": [1.0, 1.0], "eps": eps,
                        "y": [[3.0 / rms, 4.0 / rms]]},
        "rope_tables_s4_d8": {"seq": 4, "head_dim": 8, "base": 10000.0, "cos": cos, "sin": sin},
        "rope_rotate_pos3_d8": {
            "x": vec, "position": 3,
            "neox": rotate64(vec, cos[3], sin[3], "neox"),
            "interleaved": rotate64(vec, cos[3], sin[3], "interleaved"),
        },
        "silu": {"g": silu_points, "silu": [g / (1.0 + math.exp(-g)) for g in silu_points]},
    }


def reference_golden() -> dict:
    text = (REFERENCE / "docs" / "EXTENDING.md").read_text()
    line = re.search(r"rmsnorm_wrong: max_error=([0-9.e+-]+) > budget=([0-9.e+-]+) \(([0-9.]+) ulps\)", text)
    keys = {}
    for dt in ("fp16", "bf16"):
        doc = json.loads((REFERENCE / "reports" / "rtx3070" / f"selected_config_{dt}.json").read_text())
        keys[dt] = {"parameters": doc["parameters"],
                    "shape_keys": {op: rec["shape_key"] for op, rec in doc["operations"].items()}}
    return {
        "extending_rejection": {
            "source": "docs/EXTENDING.md:153-175",
            "inputs": "torch.manual_seed(0); x = torch.randn(4096, 2048); weight = torch.randn(2048); fp32",
            "wrong_kernel": "x * rsqrt(mean(|x|) + eps) * w (mean absolute value instead of RMS)",
            "max_error": line.group(1), "budget": line.group(2), "ulps": line.group(3),
        },
        "selected_config_shape_keys": {"source": "reports/rtx3070/selected_config_{fp16,bf16}.json", **keys},
        "ulp_known_answers": {
            "source": "tests/test_tolerance.py:21-27",
            "cases": [["bfloat16", 5.19, 0.03125], ["bfloat16", 1.0, 0.0078125],
                      ["float16", 5.19, 0.00390625], ["float32", 5.19, 2.0 ** 2 * 2.0 ** -23]],
        },
    }


if __name__ == "__main__":
    (HERE / "known_answers.json").write_text(json.dumps(known_answers(), indent=1) + "\n")
    (HERE / "reference_golden.json").write_text(json.dumps(reference_golden(), indent=1) + "\n")
    print("wrote", HERE / "known_answers.json", HERE / "reference_golden.json")
