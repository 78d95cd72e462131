"""Randomised GPU parity sweep: seeded random shapes, padded strides, dtypes
and weight / table dtypes for every HIP kernel, each case against the numpy
oracle (at most 2 ulp of max|ref| for fp16/bf16, 4 for fp32; the rounded
residual sum bit for bit). Deterministic: the cases come from fixed seeds,
4-6 per test by default; AKO_RANDOM_SEEDS=N runs seeds 0..N-1 of each for a
wider sweep.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
from ako_amd.ops.rope_hip import rope_hip, rope_qk_cache_hip
from ako_amd.ops.rope_ref import build_rope_tables
from ako_amd.ops.swiglu_hip import swiglu_hip
from oracle import ops as oracle
from tests._util import NAMES, to_np

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]
DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
MAX_ULPS = {torch.float16: 2.0, torch.bfloat16: 2.0, torch.float32: 4.0}


def seeds(default: int) -> range:
    """Seeds 0..default-1, or 0..AKO_RANDOM_SEEDS-1 when that is set."""
    return range(int(os.environ.get("AKO_RANDOM_SEEDS", default)))


def _check(expected: np.ndarray, got: torch.Tensor, dtype: torch.dtype, case: str) -> None:
    rep = oracle.gate(expected, to_np(got), NAMES[dtype])
    assert rep["passed"] and rep["err_ulps"] <= MAX_ULPS[dtype], (case, rep)


def _padded(rows: int, width: int, pad: int, dtype: torch.dtype, gen: torch.Generator, scale=1.0, shift=0.0):
    base = (torch.randn(rows, width + pad, generator=gen, device=DEV) * scale + shift).to(dtype)
    return base[:, :width]


@pytest.mark.parametrize("seed", seeds(6))
def test_rmsnorm_random_cases(seed: int) -> None:
    rng = np.random.default_rng(1000 + seed)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    for _ in range(12):
        dtype = DTYPES[rng.integers(3)]
        rows = int(rng.choice([1, 2, 3, 17, 64, 257]))
        hidden = int(rng.choice([1, 7, 64, 100, 511, 1024, 2050, 4096, 8191, 16384, 33000]))
        pad = int(rng.choice([0, 0, 8, 3]))
        scale = float(rng.choice([0.01, 1.0, 50.0]))
        w_fp32 = dtype != torch.float32 and rng.random() < 0.3
        x = _padded(rows, hidden, pad, dtype, gen, scale=scale)
        r = _padded(rows, hidden, pad, dtype, gen)
        w = (torch.randn(hidden, generator=gen, device=DEV) * 0.1 + 1.0).to(torch.float32 if w_fp32 else dtype)
        case = f"rows={rows} hidden={hidden} pad={pad} {dtype} w_fp32={w_fp32} scale={scale}"
        wname = "float32" if w_fp32 else NAMES[dtype]
        _check(oracle.rmsnorm(to_np(x), to_np(w), 1e-6, dtype=NAMES[dtype], w_dtype=wname),
               rmsnorm_hip(x, w, 1e-6), dtype, case)
        y, s = rmsnorm_residual_hip(x, r, w, 1e-6)
        ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), 1e-6, dtype=NAMES[dtype], w_dtype=wname)
        np.testing.assert_array_equal(to_np(s), es, err_msg=case)
        _check(ey, y, dtype, case)


@pytest.mark.parametrize("seed", seeds(4))
def test_rmsnorm_pipelined_random_cases(seed: int) -> None:
    """Launches of many full rows (the persistent pipelined kernel's domain),
    with random row counts, padded strides, weight dtypes and pipelined grid
    settings (key 9: default or forced; key 10: workgroups per CU; key 5: row
    order), against the oracle on a seeded sample of rows (rows are computed
    independently, so sampled rows check the launch)."""
    from ako_amd import _native

    rng = np.random.default_rng(5000 + seed)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    widths = {torch.float32: [2048, 4096], torch.float16: [4096, 8192], torch.bfloat16: [4096, 8192]}
    try:
        for _ in range(4):
            dtype = DTYPES[rng.integers(3)]
            rows = int(rng.choice([257, 1000, 4099, 9001, 16500]))
            hidden = int(rng.choice(widths[dtype]))
            pad = int(rng.choice([0, 8, 64]))
            w_fp32 = dtype != torch.float32 and rng.random() < 0.3
            pipeline, per_cu, order = int(rng.choice([0, 2])), int(rng.choice([0, 1, 2, 3, 5])), int(rng.choice([0, 1]))
            _native.set_tuning(0, 9, pipeline)
            _native.set_tuning(0, 10, per_cu)
            _native.set_tuning(0, 5, order)
            x = _padded(rows, hidden, pad, dtype, gen)
            r = _padded(rows, hidden, pad, dtype, gen)
            w = (torch.randn(hidden, generator=gen, device=DEV) * 0.1 + 1.0).to(torch.float32 if w_fp32 else dtype)
            pick = np.unique(np.concatenate([[0, rows - 1], rng.choice(rows, size=62, replace=False)]))
            idx = torch.as_tensor(pick, device=DEV)
            case = (f"rows={rows} hidden={hidden} pad={pad} {dtype} w_fp32={w_fp32} "
                    f"pipeline={pipeline} per_cu={per_cu} order={order}")
            wname = "float32" if w_fp32 else NAMES[dtype]
            xs, rs, wn = to_np(x[idx]), to_np(r[idx]), to_np(w)
            _check(oracle.rmsnorm(xs, wn, 1e-6, dtype=NAMES[dtype], w_dtype=wname),
                   rmsnorm_hip(x, w, 1e-6)[idx], dtype, case)
            y, s = rmsnorm_residual_hip(x, r, w, 1e-6)
            ey, es = oracle.rmsnorm_residual(xs, rs, wn, 1e-6, dtype=NAMES[dtype], w_dtype=wname)
            np.testing.assert_array_equal(to_np(s[idx]), es, err_msg=case)
            _check(ey, y[idx], dtype, case)
    finally:
        for key in (5, 9, 10):
            _native.set_tuning(0, key, 0)


@pytest.mark.parametrize("seed", seeds(6))
def test_rope_random_cases(seed: int) -> None:
    from ako_amd import _native

    rng = np.random.default_rng(2000 + seed)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    for _ in range(10):
        dtype = DTYPES[rng.integers(3)]
        tdtype = DTYPES[rng.integers(3)]
        style = str(rng.choice(["neox", "interleaved"]))
        b, s = int(rng.choice([1, 2, 5])), int(rng.choice([1, 3, 64, 130]))
        h, d = int(rng.choice([1, 3, 8, 32])), int(rng.choice([2, 6, 16, 64, 96, 128, 256]))
        offset = int(rng.choice([0, 7, 1000]))
        full = (torch.randn(b, s, h + 2, d, generator=gen, device=DEV)).to(dtype)
        x = full[:, :, 1:h + 1]  # a strided head slice
        cos, sin = build_rope_tables(s, d, offset=offset, device=DEV)
        cos, sin = cos.to(tdtype), sin.to(tdtype)
        # Wavefronts per workgroup (0: the default); 2-16 leave spare
        # wavefronts in the last workgroup, which must write nothing.
        per_block = int(rng.choice([0, 1, 2, 4, 8, 16]))
        case = (f"b={b} s={s} h={h} d={d} {style} {dtype} tables {tdtype} offset={offset} "
                f"waves/workgroup={per_block}")
        try:
            _native.set_tuning(1, 1, per_block)
            _check(oracle.rope(to_np(x), to_np(cos), to_np(sin), style, dtype=NAMES[dtype],
                               table_dtype=NAMES[tdtype]),
                   rope_hip(x, cos, sin, style), dtype, case)
        finally:
            _native.set_tuning(1, 1, 0)


@pytest.mark.parametrize("seed", seeds(4))
def test_rope_qk_cache_random_cases(seed: int) -> None:
    rng = np.random.default_rng(3000 + seed)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    for _ in range(8):
        dtype = DTYPES[rng.integers(3)]
        style = str(rng.choice(["neox", "interleaved"]))
        b, s = int(rng.choice([1, 2])), int(rng.choice([1, 4, 33]))
        hkv = int(rng.choice([1, 2, 8]))
        hq = hkv * int(rng.choice([1, 4]))
        d = int(rng.choice([6, 64, 128]))
        cache_len = s + int(rng.choice([0, 5, 100]))
        pos = int(rng.integers(0, cache_len - s + 1))
        q = torch.randn(b, s, hq, d, generator=gen, device=DEV).to(dtype)
        k = torch.randn(b, s, hkv, d, generator=gen, device=DEV).to(dtype)
        v = torch.randn(b, s, hkv, d, generator=gen, device=DEV).to(dtype)
        kc = torch.randn(b, hkv, cache_len, d, generator=gen, device=DEV).to(dtype)
        vc = torch.randn(b, hkv, cache_len, d, generator=gen, device=DEV).to(dtype)
        cos, sin = build_rope_tables(cache_len, d, device=DEV)
        eq, ek, ev = oracle.rope_qk_cache(to_np(q), to_np(k), to_np(v), to_np(cos), to_np(sin), pos, to_np(kc),
                                          to_np(vc), style, dtype=NAMES[dtype])
        case = f"b={b} s={s} hq={hq} hkv={hkv} d={d} cache={cache_len} pos={pos} {style} {dtype}"
        q_out = rope_qk_cache_hip(q, k, v, cos, sin, torch.tensor([pos], device=DEV), kc, vc, style)
        _check(eq, q_out, dtype, case)
        _check(ek, kc, dtype, case)
        np.testing.assert_array_equal(to_np(vc), ev, err_msg=case)


@pytest.mark.parametrize("seed", seeds(4))
def test_swiglu_random_cases(seed: int) -> None:
    rng = np.random.default_rng(4000 + seed)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    for _ in range(10):
        dtype = DTYPES[rng.integers(3)]
        rows = int(rng.choice([1, 3, 16, 100]))
        n = int(rng.choice([1, 5, 64, 1000, 4097, 14336]))
        pad = int(rng.choice([0, 0, 8, 1]))
        scale = float(rng.choice([1.0, 8.0, 40.0]))
        g = _padded(rows, n, pad, dtype, gen, scale=scale)
        u = _padded(rows, n, pad, dtype, gen)
        case = f"rows={rows} n={n} pad={pad} {dtype} scale={scale}"
        _check(oracle.swiglu(to_np(g), to_np(u), dtype=NAMES[dtype]), swiglu_hip(g, u), dtype, case)
