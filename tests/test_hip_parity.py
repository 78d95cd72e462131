"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Every case checks two things on identical seeded inputs:

* the repository's own gate against the unfused PyTorch reference run on the
  same device (``atol + rtol(dtype) * max|ref|``, ``ako_amd.validation``), on the
  whole output, at the BASELINE.json sizes;
* agreement with the numpy oracle (``oracle.ops``) in ulps of ``max|ref|``:
  at most 2 ulp for fp16/bf16 and 4 ulp for fp32 (the north-star target), on
  the whole output where the oracle finishes in seconds and on a seeded
  sample of rows otherwise (rows are computed independently, so sampled rows
  of a full-size launch check that launch). Integer-like results (the rounded
  residual sum) must match the oracle bit for bit.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref, rmsnorm_residual_ref
from ako_amd.ops.rope_hip import rope_hip, rope_qk_cache_hip, rope_qk_hip
from ako_amd.ops.rope_ref import build_rope_tables, rope_ref
from ako_amd.ops.swiglu_hip import swiglu_hip
from ako_amd.ops.swiglu_ref import swiglu_ref
from ako_amd.validation.numerical import error_budget, max_abs_error_any
from oracle import ops as oracle
from tests._util import NAMES, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

MAX_ULPS = {torch.float16: 2.0, torch.bfloat16: 2.0, torch.float32: 4.0}
DEV = "cuda"


def grandn(shape, dtype, seed, *, scale=1.0, shift=0.0) -> torch.Tensor:
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV) * scale + shift).to(dtype)


def sample_rows(n_rows: int, k: int = 256, seed: int = 0) -> np.ndarray:
    if n_rows <= k:
        return np.arange(n_rows)
    rng = np.random.default_rng(seed)
    picked = rng.choice(n_rows, size=k - 2, replace=False)
    return np.unique(np.concatenate([[0, n_rows - 1], picked]))


def assert_gate(ref, out) -> None:
    err = max_abs_error_any(ref, out)
    budget = error_budget(ref)
    assert err <= budget, f"gate: max_error={err:.3e} > budget={budget:.3e}"


def assert_rope_exact(expected: np.ndarray, got: np.ndarray, dtype: torch.dtype) -> None:
    """RoPE rounds the same fp32 products and sums as the oracle (the library
    is built without contraction): every element bit for bit, plus the gate."""
    assert_oracle(expected, got, dtype)
    np.testing.assert_array_equal(got, expected)


def assert_oracle(expected: np.ndarray, got: np.ndarray, dtype: torch.dtype) -> dict:
    report = oracle.gate(expected, got, NAMES[dtype])
    assert report["passed"], report
    assert report["err_ulps"] <= MAX_ULPS[dtype], report
    return report


# ----------------------------------------------------------------------- RMSNorm --

RMS_GRID = [(rows, h) for h in (4096, 8192, 16384) for rows in (1, 32, 16384)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden", RMS_GRID)
def test_rmsnorm_config2(rows: int, hidden: int, dtype: torch.dtype) -> None:
    x = grandn((rows, hidden), dtype, 0)
    w = grandn((hidden,), dtype, 1, scale=0.1, shift=1.0)
    y = rmsnorm_hip(x, w, 1e-6)
    torch.cuda.synchronize()
    assert y.shape == x.shape and y.dtype == dtype
    assert_gate(rmsnorm_ref(x, w, 1e-6), y)
    idx = sample_rows(rows)
    sel = torch.as_tensor(idx, device=DEV)
    expected = oracle.rmsnorm(to_np(x[sel]), to_np(w), 1e-6, dtype=NAMES[dtype])
    assert_oracle(expected, to_np(y[sel]), dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden", RMS_GRID)
def test_rmsnorm_residual_config2(rows: int, hidden: int, dtype: torch.dtype) -> None:
    x = grandn((rows, hidden), dtype, 0)
    r = grandn((rows, hidden), dtype, 2)
    w = grandn((hidden,), dtype, 1, scale=0.1, shift=1.0)
    y, s = rmsnorm_residual_hip(x, r, w, 1e-6)
    torch.cuda.synchronize()
    assert_gate(rmsnorm_residual_ref(x, r, w, 1e-6), (y, s))
    idx = sample_rows(rows)
    sel = torch.as_tensor(idx, device=DEV)
    ey, es = oracle.rmsnorm_residual(to_np(x[sel]), to_np(r[sel]), to_np(w), 1e-6, dtype=NAMES[dtype])
    np.testing.assert_array_equal(to_np(s[sel]), es)  # the rounded sum is exact
    assert_oracle(ey, to_np(y[sel]), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 128, 1024), (2, 128, 512), (1, 2048, 4096), (3, 100),
                                   (2, 8448), (5, 1), (4, 7), (3, 65_536), (2, 65_544), (2, 140_000), (1, 262_144)])
def test_rmsnorm_shapes_dtypes(shape, dtype: torch.dtype) -> None:
    """Reference test shapes, ragged widths (scalar path), rows wider than the
    register budget (two-pass path), every dtype."""
    x = grandn(shape, dtype, 3, scale=3.0)
    w = grandn(shape[-1:], dtype, 4, scale=0.1, shift=1.0)
    y = rmsnorm_hip(x, w)
    assert_gate(rmsnorm_ref(x, w), y)
    assert_oracle(oracle.rmsnorm(to_np(x), to_np(w), dtype=NAMES[dtype]), to_np(y), dtype)
    r = grandn(shape, dtype, 5)
    y2, s2 = rmsnorm_residual_hip(x, r, w)
    ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), dtype=NAMES[dtype])
    np.testing.assert_array_equal(to_np(s2), es)
    assert_oracle(ey, to_np(y2), dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rmsnorm_fp32_weight_and_strided_rows(dtype: torch.dtype) -> None:
    base = grandn((64, 4096 + 64), dtype, 6)
    x = base[:, :4096]  # rows 4160 elements apart, no copy
    w = grandn((4096,), torch.float32, 7, scale=0.1, shift=1.0)
    y = rmsnorm_hip(x, w)
    expected = oracle.rmsnorm(to_np(x), to_np(w), dtype=NAMES[dtype], w_dtype="float32")
    assert_oracle(expected, to_np(y), dtype)
    # Padded stride but a width that is not a multiple of the packet: scalar tail lanes.
    xt = base[:, :4093]
    wt = grandn((4093,), dtype, 8, scale=0.1, shift=1.0)
    assert_oracle(oracle.rmsnorm(to_np(xt), to_np(wt), dtype=NAMES[dtype]), to_np(rmsnorm_hip(xt, wt)), dtype)
    # Misaligned start (offset by one element): the scalar path.
    xm = base.reshape(-1)[1: 1 + 8 * 4096].view(8, 4096)
    assert_oracle(oracle.rmsnorm(to_np(xm), to_np(w), dtype=NAMES[dtype], w_dtype="float32"),
                  to_np(rmsnorm_hip(xm, w)), dtype)


def test_rmsnorm_every_register_shape() -> None:
    """Each instantiated (waves per row, packets per lane) shape is correct."""
    from ako_amd import _native

    x = grandn((37, 4096), torch.bfloat16, 9)
    r = grandn((37, 4096), torch.bfloat16, 10)
    w = grandn((4096,), torch.bfloat16, 11, scale=0.1, shift=1.0)
    expected = oracle.rmsnorm(to_np(x), to_np(w), dtype="bfloat16")
    ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), dtype="bfloat16")
    w32 = w.float()
    expected32 = oracle.rmsnorm(to_np(x), to_np(w32), dtype="bfloat16", w_dtype="float32")
    shapes = [(1, 8), (2, 4), (2, 8), (4, 2), (4, 4), (4, 8), (8, 1), (8, 2), (8, 4), (8, 8), (16, 1), (16, 2), (16, 4), (16, 8)]
    try:
        for wpr, vpt in shapes:
            _native.set_tuning(0, 1, wpr)
            _native.set_tuning(0, 2, vpt)
            # One- and two-packet shapes also come with early weight loads
            # (key 8: 1 = late, 2 = early); the others ignore the key.
            for early in ((1, 2) if vpt <= 2 else (0,)):
                _native.set_tuning(0, 8, early)
                assert_oracle(expected, to_np(rmsnorm_hip(x, w)), torch.bfloat16)
                assert_oracle(expected32, to_np(rmsnorm_hip(x, w32)), torch.bfloat16)
                y, s = rmsnorm_residual_hip(x, r, w)
                np.testing.assert_array_equal(to_np(s), es)
                assert_oracle(ey, to_np(y), torch.bfloat16)
        for key in (1, 2, 8):
            _native.set_tuning(0, key, 0)
        _native.set_tuning(0, 3, 1)  # force the two-pass kernel
        assert_oracle(expected, to_np(rmsnorm_hip(x, w)), torch.bfloat16)
    finally:
        for key in (1, 2, 3, 8):
            _native.set_tuning(0, key, 0)


@pytest.mark.parametrize("rows", [127, 128, 1000, 2051])
def test_rmsnorm_xcd_row_orders_cover_every_row(rows: int) -> None:
    """Every row order maps workgroups onto rows one to one.

    Row counts straddle the 128-workgroup threshold of the default chunked
    order, and 1000 / 2051 leave partial runs and trailing blocks. Rows are
    independent, so any order must give bit-identical outputs to block order.
    """
    from ako_amd import _native

    x = grandn((rows, 2048), torch.float16, 30)
    r = grandn((rows, 2048), torch.float16, 31)
    w = grandn((2048,), torch.float16, 32, scale=0.1, shift=1.0)
    ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), dtype="float16")
    try:
        _native.set_tuning(0, 5, 1)
        base_y, base_s = rmsnorm_residual_hip(x, r, w)
        base_p = rmsnorm_hip(x, w)
        np.testing.assert_array_equal(to_np(base_s), es)
        assert_oracle(ey, to_np(base_y), torch.float16)
        for order, chunk in ((0, 0), (2, 0), (2, 1), (2, 3), (2, 16), (2, 100000)):
            _native.set_tuning(0, 5, order)
            _native.set_tuning(0, 6, chunk)
            y, s = rmsnorm_residual_hip(x, r, w)
            assert torch.equal(y, base_y) and torch.equal(s, base_s), (order, chunk)
            assert torch.equal(rmsnorm_hip(x, w), base_p), (order, chunk)
    finally:
        for key in (5, 6):
            _native.set_tuning(0, key, 0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows", [31, 33, 127, 130, 257, 1000, 2051])
def test_rmsnorm_wide_rows_xcd_runs_cover_every_row(rows: int, dtype: torch.dtype) -> None:
    """Rows of 16384 half elements go to the XCDs in runs: residual rows in
    runs of 16 from 128 workgroups up (runs of 8 from 64, block order below),
    plain rows in runs of 4 from 32 workgroups up (block order below). Row
    counts straddle those thresholds and the 256-row switch to write-through
    stores, and 1000 / 2051 leave partial runs and trailing blocks; the
    default order must give bit-identical outputs to block order, which is
    checked against the oracle on the first and last rows."""
    from ako_amd import _native

    x = grandn((rows, 16384), dtype, 40)
    r = grandn((rows, 16384), dtype, 41)
    w = grandn((16384,), dtype, 42, scale=0.1, shift=1.0)
    name = NAMES[dtype]
    try:
        _native.set_tuning(0, 5, 1)
        base_y, base_s = rmsnorm_residual_hip(x, r, w)
        base_p = rmsnorm_hip(x, w)
    finally:
        _native.set_tuning(0, 5, 0)
    y, s = rmsnorm_residual_hip(x, r, w)
    assert torch.equal(y, base_y) and torch.equal(s, base_s)
    p = rmsnorm_hip(x, w)
    assert torch.equal(p, base_p)
    n = min(48, rows)
    for sl in (slice(0, n), slice(rows - n, rows)):
        ey, es = oracle.rmsnorm_residual(to_np(x[sl]), to_np(r[sl]), to_np(w), dtype=name)
        np.testing.assert_array_equal(to_np(s[sl]), es)
        assert_oracle(ey, to_np(y[sl]), dtype)
        assert_oracle(oracle.rmsnorm(to_np(x[sl]), to_np(w), dtype=name), to_np(p[sl]), dtype)


@pytest.mark.parametrize("cap", [1, 3, 7, 64])
def test_rmsnorm_split_launches_match_one_launch(cap: int) -> None:
    """Problems past the per-launch workgroup cap run as several launches from
    row offsets; with the cap lowered (key 7) the split path must reproduce the
    single launch bit for bit, for packed-row, wide-row and two-pass kernels."""
    from ako_amd import _native

    cases = [(301, 256), (259, 4096), (97, 140_000)]  # 4 rows per block, XCD-ordered wide rows, two-pass
    try:
        _native.set_tuning(0, 9, 1)  # one row per workgroup (the persistent kernel never splits)
        for rows, hidden in cases:
            x = grandn((rows, hidden), torch.bfloat16, 33)
            r = grandn((rows, hidden), torch.bfloat16, 34)
            w = grandn((hidden,), torch.bfloat16, 35, scale=0.1, shift=1.0)
            _native.set_tuning(0, 7, 0)
            want_p = rmsnorm_hip(x, w)
            want_y, want_s = rmsnorm_residual_hip(x, r, w)
            _native.set_tuning(0, 7, cap)
            assert torch.equal(rmsnorm_hip(x, w), want_p), (rows, hidden, cap)
            y, s = rmsnorm_residual_hip(x, r, w)
            assert torch.equal(y, want_y) and torch.equal(s, want_s), (rows, hidden, cap)
        ey = oracle.rmsnorm(to_np(x), to_np(w), dtype="bfloat16")
        assert_oracle(ey, to_np(rmsnorm_hip(x, w)), torch.bfloat16)
    finally:
        _native.set_tuning(0, 7, 0)
        _native.set_tuning(0, 9, 0)


@pytest.mark.parametrize("hidden,rows", [(4096, 9000), (8192, 4100), (16384, 300)])
def test_rmsnorm_padded_output_strides_through_the_abi(hidden, rows) -> None:
    """Outputs with padded row strides, through the C ABI, at launch sizes the
    pipelined kernel (4096 and 8192) and the one-packet load groups (bf16
    16384) take: the padding is never written and the rows equal the
    contiguous result."""
    from ako_amd import _native

    lib = _native.load()
    dtype, pad = torch.bfloat16, 64
    x = grandn((rows, hidden), dtype, 90)
    r = grandn((rows, hidden), dtype, 91)
    w = grandn((hidden,), dtype, 92, scale=0.1, shift=1.0)
    want_y, want_s = rmsnorm_residual_hip(x, r, w)
    want_p = rmsnorm_hip(x, w)
    sentinel = -7.0
    y = torch.full((rows, hidden + pad), sentinel, dtype=dtype, device=DEV)
    s_ = torch.full((rows, hidden + pad), sentinel, dtype=dtype, device=DEV)
    p = torch.full((rows, hidden + pad), sentinel, dtype=dtype, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    code = _native.DTYPE_CODES[dtype]
    assert lib.ako_rmsnorm_residual_fwd(x.data_ptr(), r.data_ptr(), w.data_ptr(), y.data_ptr(), s_.data_ptr(),
                                        rows, hidden, hidden, hidden, hidden + pad, hidden + pad, 1e-6, code, code,
                                        stream) == 0
    assert lib.ako_rmsnorm_fwd(x.data_ptr(), w.data_ptr(), p.data_ptr(), rows, hidden, hidden, hidden + pad, 1e-6,
                               code, code, stream) == 0
    for out, want in ((y, want_y), (s_, want_s), (p, want_p)):
        assert torch.equal(out[:, :hidden], want)
        assert bool((out[:, hidden:] == sentinel).all())


@pytest.mark.parametrize("dtype,w_dtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                           (torch.float16, torch.float16)])
def test_rmsnorm_residual_load_groups_match(dtype, w_dtype) -> None:
    """The residual (16 wavefronts, 2 packets) rows with both packets loaded
    as one group (key 11 = 1) and one packet at a time (key 11 = 2): the same
    sums in the same order, so bit-identical outputs, at a decode-sized and a
    many-row launch; the default choice against the oracle."""
    from ako_amd import _native

    h = 16384
    try:
        for rows in (33, 300):
            x = grandn((rows, h), dtype, 60 + rows)
            r = grandn((rows, h), dtype, 61 + rows)
            w = grandn((h,), w_dtype, 62, scale=0.1, shift=1.0)
            outs = {}
            for key in (1, 2, 0):
                _native.set_tuning(0, 11, key)
                outs[key] = rmsnorm_residual_hip(x, r, w)
            assert all(torch.equal(a, b) for a, b in zip(outs[1], outs[2])), rows
            assert all(torch.equal(a, b) for a, b in zip(outs[0], outs[1])), rows
            ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), dtype=NAMES[dtype], w_dtype=NAMES[w_dtype])
            np.testing.assert_array_equal(to_np(outs[0][1]), es)
            assert_oracle(ey, to_np(outs[0][0]), dtype)
    finally:
        _native.set_tuning(0, 11, 0)


# (dtype, weight dtype, hidden, row stride or None): rows on the (16, 2) shape,
# full (16384 half / 8192 fp32 elements) and with idle lanes (9000, 12000), and
# residual rows on the (16, 1) shape (8192 half elements; 7000 with idle lanes).
WRITE_THROUGH_CASES = [
    (torch.float16, torch.float16, 16384, None),
    (torch.bfloat16, torch.float32, 16384, 16448),
    (torch.float16, torch.float16, 12000, None),
    (torch.bfloat16, torch.bfloat16, 9000, 9008),
    (torch.float32, torch.float32, 8192, None),
    (torch.float16, torch.float16, 8192, None),
    (torch.bfloat16, torch.bfloat16, 7000, 7008),
]


@pytest.mark.parametrize("dtype,w_dtype,h,stride", WRITE_THROUGH_CASES)
def test_rmsnorm_write_through_stores_match(dtype, w_dtype, h, stride) -> None:
    """Rows on the (16, 2) and (16, 1) shapes stored write-through (key 12 = 2, buffer
    stores with sc1 nt on a resource covering the row) and with plain
    non-temporal stores (key 12 = 1), residual rows with either load grouping:
    the same values in the same places, so bit-identical outputs, also where
    lanes sit idle and where input rows are padded; the default
    (write-through from 257 rows on (16, 2), non-temporal on (16, 1)) against
    the oracle on sampled rows."""
    from ako_amd import _native

    try:
        for rows in (3, 300):
            width = stride or h
            xb = grandn((rows, width), dtype, 70 + rows)
            rb = grandn((rows, width), dtype, 71 + rows)
            x, r = xb[:, :h], rb[:, :h]
            w = grandn((h,), w_dtype, 72, scale=0.1, shift=1.0)
            outs = {}
            for wt in (1, 2, 0):
                for groups in (1, 2):
                    _native.set_tuning(0, 12, wt)
                    _native.set_tuning(0, 11, groups)
                    outs[(wt, groups)] = (rmsnorm_hip(x, w), *rmsnorm_residual_hip(x, r, w))
            base = outs[(1, 1)]
            for key, got in outs.items():
                assert all(torch.equal(a, b) for a, b in zip(got, base)), (rows, key)
            idx = sample_rows(rows, 64)
            sel = torch.as_tensor(idx, device=DEV)
            wname = NAMES[w_dtype]
            assert_oracle(oracle.rmsnorm(to_np(x[sel]), to_np(w), dtype=NAMES[dtype], w_dtype=wname),
                          to_np(outs[(0, 1)][0][sel]), dtype)
            ey, es = oracle.rmsnorm_residual(to_np(x[sel]), to_np(r[sel]), to_np(w), dtype=NAMES[dtype],
                                             w_dtype=wname)
            np.testing.assert_array_equal(to_np(outs[(0, 1)][2][sel]), es)
            assert_oracle(ey, to_np(outs[(0, 1)][1][sel]), dtype)
    finally:
        _native.set_tuning(0, 11, 0)
        _native.set_tuning(0, 12, 0)


# (dtype, weight dtype, hidden, forced (waves per row, packets per lane) or None).
# Every shape with a pipelined instantiation appears; None is the default shape
# of a launch of many rows (full rows: hidden = 64 * waves * packets * E).
PIPE_CASES = [
    (torch.float16, torch.float16, 4096, None),      # plain (4, 2), residual (8, 1)
    (torch.bfloat16, torch.bfloat16, 8192, None),    # plain (8, 2), residual (16, 1)
    (torch.bfloat16, torch.float32, 16384, None),    # (16, 2), fp32 weight
    (torch.float16, torch.float16, 32768, None),     # (16, 4)
    (torch.float32, torch.float32, 2048, None),      # fp32 rows, (4, 2) / (8, 1)
    (torch.float16, torch.float32, 8192, (8, 1)),
    (torch.bfloat16, torch.bfloat16, 16384, (16, 1)),
    (torch.float32, torch.float32, 4096, (16, 1)),
]


@pytest.mark.parametrize("dtype,w_dtype,hidden,shape", PIPE_CASES,
                         ids=[f"{NAMES[d]}-{NAMES[w]}-{h}-{s}" for d, w, h, s in PIPE_CASES])
def test_rmsnorm_pipelined_kernel_matches_register_kernel(dtype, w_dtype, hidden, shape) -> None:
    """The persistent, software-pipelined kernel (key 9 = 2) against the
    one-row-per-workgroup kernel (key 9 = 1): the same arithmetic in the same
    order, so outputs must be bit-identical, for both row orders (key 5),
    several grid sizes (key 10: 1 and 3 workgroups per CU, 32 leaves most
    workgroups one row or none) and row counts with odd and even trips per
    workgroup, empty XCD ranges and a strided input. One case per dtype is
    also checked against the oracle."""
    from ako_amd import _native

    rows_list = [257, 1031, 4099] + ([16384] if hidden <= 8192 else []) if hidden <= 16384 else [257, 1031]
    try:
        if shape is not None:
            _native.set_tuning(0, 1, shape[0])
            _native.set_tuning(0, 2, shape[1])
        for rows in rows_list:
            base = grandn((rows, hidden + 64), dtype, 40 + rows)
            x = base[:, :hidden]  # row stride hidden + 64
            r = grandn((rows, hidden), dtype, 41 + rows)
            w = grandn((hidden,), w_dtype, 42, scale=0.1, shift=1.0)
            for key in (5, 10):  # left set by the previous row count's sweep
                _native.set_tuning(0, key, 0)
            _native.set_tuning(0, 9, 1)
            want_p = rmsnorm_hip(x, w)
            want_y, want_s = rmsnorm_residual_hip(x, r, w)
            if rows == rows_list[0]:
                assert_oracle(oracle.rmsnorm(to_np(x), to_np(w), dtype=NAMES[dtype], w_dtype=NAMES[w_dtype]),
                              to_np(want_p), dtype)
            # The default choice. Rows of 512 or 1024 packets go pipelined at
            # one packet per lane (when their input fits 16 KiB; plain rows
            # only with 16 rows per workgroup, as at 16384 rows) or to the
            # register kernel's one-packet residual shape: either way the
            # register kernel at (packets / 64, 1) sums in the same order.
            # Plain rows short of the row count take the register kernel's
            # own default shape.
            nvec = hidden * x.element_size() // 16
            if shape is None and nvec in (512, 1024):
                _native.set_tuning(0, 1, nvec // 64)
                _native.set_tuning(0, 2, 1)
                want_dp = rmsnorm_hip(x, w)
                want_dy, _ = rmsnorm_residual_hip(x, r, w)
                _native.set_tuning(0, 1, 0)
                _native.set_tuning(0, 2, 0)
            else:
                want_dp, want_dy = want_p, want_y
            _native.set_tuning(0, 9, 0)
            got_p = rmsnorm_hip(x, w)
            got_y, got_s = rmsnorm_residual_hip(x, r, w)
            assert torch.equal(got_y, want_dy), rows
            if shape is None and nvec in (512, 1024) and rows >= 16384:
                assert torch.equal(got_p, want_dp), rows
            else:
                assert torch.equal(got_p, want_dp) or torch.equal(got_p, want_p), rows
            assert torch.equal(got_s, want_s), rows
            if rows == rows_list[0]:
                ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), dtype=NAMES[dtype],
                                                 w_dtype=NAMES[w_dtype])
                assert_oracle(ey, to_np(got_y), dtype)
                np.testing.assert_array_equal(to_np(got_s), es)
                assert_oracle(oracle.rmsnorm(to_np(x), to_np(w), dtype=NAMES[dtype], w_dtype=NAMES[w_dtype]),
                              to_np(got_p), dtype)
            _native.set_tuning(0, 9, 2)
            for order in (0, 1):
                _native.set_tuning(0, 5, order)
                for per_cu in (0, 1, 3, 32):
                    _native.set_tuning(0, 10, per_cu)
                    tag = (rows, order, per_cu)
                    assert torch.equal(rmsnorm_hip(x, w), want_p), tag
                    y, s = rmsnorm_residual_hip(x, r, w)
                    assert torch.equal(s, want_s), tag
                    assert torch.equal(y, want_y), tag
    finally:
        for key in (1, 2, 5, 9, 10):
            _native.set_tuning(0, key, 0)


def test_rmsnorm_empty_and_errors() -> None:
    w = torch.ones(64, device=DEV, dtype=torch.float16)
    empty = torch.empty(0, 64, device=DEV, dtype=torch.float16)
    assert rmsnorm_hip(empty, w).shape == (0, 64)
    with pytest.raises(ValueError, match="weight"):
        rmsnorm_hip(torch.ones(4, 64, device=DEV, dtype=torch.float16), torch.ones(32, device=DEV))
    with pytest.raises(ValueError, match="GPU"):
        rmsnorm_hip(torch.ones(4, 64), torch.ones(64))


# -------------------------------------------------------------------------- RoPE --

ROPE_BS = [(1, 1), (64, 1), (4, 2048)]


def _half_ulp_distance(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in ulps between two arrays of 16-bit float patterns."""
    def ordered(bits):
        b = bits.astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    return np.abs(ordered(a_bits) - ordered(b_bits))


@pytest.mark.parametrize("seq", [1, 640, 2048])
def test_device_built_tables_match_the_oracle(seq: int) -> None:
    """``build_rope_tables(device="cuda")`` against ``oracle.rope_tables``.

    fp32: the GPU's ``pow`` (inv_freq) and ``cos``/``sin`` are 1-2 ulp
    functions, and an inv_freq 1 ulp off moves the angle ``pos * inv_freq`` by
    about ``|angle| * 2^-23``, which the table value inherits in absolute
    terms. The bound is therefore 2 ulp of 1 plus 3 angle ulps:
    ``2 * 2^-24 + 3 * |angle| * 2^-23``. fp16/bf16 tables are the fp32 tables
    narrowed on the device (bit for bit), and within one ulp of the oracle's
    narrowed tables plus the same angle term.
    """
    d = 128
    cos, sin = build_rope_tables(seq, d, device=DEV)
    assert cos.dtype == torch.float32 and cos.shape == (seq, d // 2) and cos.is_cuda
    ec, es = oracle.rope_tables(seq, d)
    # The angles as the oracle forms them (fp32 rounded once per step).
    half = d // 2
    inv = np.float32(1.0) / np.power(np.float64(10000.0),
                                     (np.arange(half, dtype=np.float32) * 2 / d).astype(np.float64)).astype(np.float32)
    angles = np.abs(np.outer(np.arange(seq, dtype=np.float32), inv).astype(np.float64))
    bound = 2 * 2.0**-24 + 3 * angles * 2.0**-23
    for got, exp in ((cos, ec), (sin, es)):
        diff = np.abs(got.cpu().numpy().astype(np.float64) - exp.astype(np.float64))
        assert np.all(diff <= bound), (float(diff.max()), float((diff / bound).max()))
    # Known values: position 0 is the identity, position 1 rotates pair 0 by 1 rad.
    assert torch.all(cos[0] == 1.0) and torch.all(sin[0] == 0.0)
    if seq > 1:
        assert abs(float(cos[1, 0]) - math.cos(1.0)) <= 2 * 2.0**-24
        assert abs(float(sin[1, 0]) - math.sin(1.0)) <= 2 * 2.0**-24
    # Offsets are a shift of the same tables (same fp32 operations per row).
    if seq > 8:
        oc, osn = build_rope_tables(8, d, offset=seq - 8, device=DEV)
        assert torch.equal(oc, cos[-8:]) and torch.equal(osn, sin[-8:])
    for dtype in (torch.float16, torch.bfloat16):
        hc, hs = build_rope_tables(seq, d, device=DEV, dtype=dtype)
        assert torch.equal(hc, cos.to(dtype)) and torch.equal(hs, sin.to(dtype))
        name = NAMES[dtype]
        unit = {torch.float16: 2.0**-11, torch.bfloat16: 2.0**-8}[dtype]
        for got, exp32 in ((hc, ec), (hs, es)):
            exp = oracle.round_to(exp32, name)
            g, e = to_np(got), exp
            close = _half_ulp_distance(g.view(np.uint16), e.view(np.uint16)) <= 1
            # Where the fp32 values straddle a rounding boundary by more than
            # the angle term, one more ulp is allowed.
            near = np.abs(got.float().cpu().numpy().astype(np.float64) - exp32.astype(np.float64)) <= \
                unit + bound
            assert np.all(close | near)


@pytest.mark.parametrize("style", ["neox", "interleaved"])
@pytest.mark.parametrize("table_dtype", ["x", torch.float32])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("batch,seq", ROPE_BS)
def test_rope_config3(batch: int, seq: int, dtype, table_dtype, style: str) -> None:
    tdt = dtype if table_dtype == "x" else table_dtype
    cos, sin = build_rope_tables(seq, 128, base=10000.0, device=DEV, dtype=torch.float32)
    cos, sin = cos.to(tdt), sin.to(tdt)
    q = grandn((batch, seq, 32, 128), dtype, 0)
    k = grandn((batch, seq, 8, 128), dtype, 1)
    for t in (q, k):
        out = rope_hip(t, cos, sin, style)
        assert_gate(rope_ref(t, cos, sin, style), out)
        expected = oracle.rope(to_np(t), to_np(cos), to_np(sin), style, dtype=NAMES[dtype],
                               table_dtype=NAMES[tdt])
        assert_rope_exact(expected, to_np(out), dtype)
    qo, ko = rope_qk_hip(q, k, cos, sin, style)
    torch.testing.assert_close(qo, rope_hip(q, cos, sin, style), rtol=0, atol=0)
    torch.testing.assert_close(ko, rope_hip(k, cos, sin, style), rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("style", ["neox", "interleaved"])
@pytest.mark.parametrize("shape", [(2, 128, 8, 64), (1, 2048, 32, 128), (2, 6, 3, 8),
                                   (2, 5, 3, 6), (1, 9, 4, 96), (3, 4, 2, 256), (1, 1025, 12, 96)])
def test_rope_shapes(shape, style: str, dtype) -> None:
    """Reference test shapes plus head dims on the scalar path (6) and odd packet counts (96);
    (1, 1025, 12, 96) is a four-wavefront-workgroup launch whose last workgroup holds
    two spare wavefronts, with idle lanes in every wavefront."""
    x = grandn(shape, dtype, 12)
    cos, sin = build_rope_tables(shape[1], shape[-1], device=DEV)
    out = rope_hip(x, cos, sin, style=style)
    assert_gate(rope_ref(x, cos, sin, style), out)
    assert_rope_exact(oracle.rope(to_np(x), to_np(cos), to_np(sin), style, dtype=NAMES[dtype]),
                  to_np(out), dtype)


@pytest.mark.parametrize("style", ["neox", "interleaved"])
def test_rope_strided_views(style: str) -> None:
    """q/k sliced out of a fused QKV projection are rotated without a copy."""
    b, s, hq, hk, d = 2, 16, 8, 2, 128
    qkv = grandn((b, s, (hq + 2 * hk) * d), torch.bfloat16, 13)
    q = qkv[..., : hq * d].view(b, s, hq, d)
    k = qkv[..., hq * d: (hq + hk) * d].view(b, s, hk, d)
    assert not q.is_contiguous()
    cos, sin = build_rope_tables(s, d, device=DEV)
    full = build_rope_tables(64, d, device=DEV)
    for t in (q, k):
        assert_rope_exact(oracle.rope(to_np(t), to_np(cos), to_np(sin), style, dtype="bfloat16"),
                      to_np(rope_hip(t, cos, sin, style)), torch.bfloat16)
    qo, ko = rope_qk_hip(q, k, cos, sin, style)
    assert_rope_exact(oracle.rope(to_np(k), to_np(cos), to_np(sin), style, dtype="bfloat16"),
                  to_np(ko), torch.bfloat16)
    # Tables sliced from a longer table (decode offset): row stride stays D/2.
    c2, s2 = full[0][10:26], full[1][10:26]
    assert_rope_exact(oracle.rope(to_np(q), to_np(c2), to_np(s2), style, dtype="bfloat16"),
                  to_np(rope_hip(q, c2, s2, style)), torch.bfloat16)


CACHE_CASES = [
    (1, 1, 32, 32, 128, 511, 640),  # configs[4] decode step: MHA, slot 511 of 640
    (2, 5, 8, 2, 128, 3, 16),       # GQA, several tokens at once
    (1, 4, 4, 4, 6, 0, 8),          # head_dim 6: the scalar kernel
    (1, 3, 2, 2, 64, 6, 8),         # the last token's slot (8) is past the cache: dropped
    (1, 512, 32, 32, 128, 0, 640),  # configs[4] prefill: 6144 wavefronts, four per workgroup
    (2, 300, 32, 8, 128, 20, 310),  # GQA prefill at an offset, the last 10 tokens past the cache
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("style", ["neox", "interleaved"])
@pytest.mark.parametrize("batch,seq,hq,hkv,d,pos,cache_len", CACHE_CASES)
def test_rope_qk_cache(batch, seq, hq, hkv, d, pos, cache_len, style: str, dtype) -> None:
    """q rotated out, k rotated and v copied into heads-major cache slots pos + s."""
    q = grandn((batch, seq, hq, d), dtype, 40)
    k = grandn((batch, seq, hkv, d), dtype, 41)
    v = grandn((batch, seq, hkv, d), dtype, 42)
    kc = grandn((batch, hkv, cache_len, d), dtype, 43)
    vc = grandn((batch, hkv, cache_len, d), dtype, 44)
    cos, sin = build_rope_tables(cache_len, d, device=DEV)
    pos_t = torch.tensor([pos], dtype=torch.int64, device=DEV)
    eq, ek, ev = oracle.rope_qk_cache(to_np(q), to_np(k), to_np(v), to_np(cos), to_np(sin), pos,
                                      to_np(kc), to_np(vc), style, dtype=NAMES[dtype])
    q_out = rope_qk_cache_hip(q, k, v, cos, sin, pos_t, kc, vc, style)
    kept = [s for s in range(seq) if pos + s < cache_len]
    dropped = [s for s in range(seq) if pos + s >= cache_len]
    untouched = [t for t in range(cache_len) if not pos <= t < pos + len(kept)]
    # RoPE rounds the oracle's own fp32 products and sums: bit for bit.
    np.testing.assert_array_equal(to_np(q_out[:, kept]), eq[:, kept])
    # Tokens past the cache: every q element NaN (never stale memory).
    assert torch.isnan(q_out[:, dropped].float()).all()
    np.testing.assert_array_equal(to_np(kc), ek)
    np.testing.assert_array_equal(to_np(vc), ev)
    # The same rotation as the one-launch pair kernel on the same table rows, bit for bit.
    n = len(kept)
    qo, ko = rope_qk_hip(q[:, :n], k[:, :n], cos[pos:pos + n], sin[pos:pos + n], style)
    assert torch.equal(q_out[:, :n], qo)
    assert torch.equal(kc[:, :, pos:pos + n], ko.transpose(1, 2))


def test_rope_qk_cache_without_values_and_rejects() -> None:
    q = grandn((1, 1, 4, 128), torch.float16, 45)
    k = grandn((1, 1, 2, 128), torch.float16, 46)
    kc = torch.zeros(1, 2, 32, 128, device=DEV, dtype=torch.float16)
    cos, sin = build_rope_tables(32, 128, device=DEV)
    pos = torch.tensor([7], dtype=torch.int64, device=DEV)
    q_out = rope_qk_cache_hip(q, k, None, cos, sin, pos, kc, None)
    qo, ko = rope_qk_hip(q, k, cos[7:8], sin[7:8])
    assert torch.equal(q_out, qo) and torch.equal(kc[:, :, 7:8], ko.transpose(1, 2))
    assert not kc[:, :, :7].any() and not kc[:, :, 8:].any()
    with pytest.raises(ValueError, match="int64"):
        rope_qk_cache_hip(q, k, None, cos, sin, pos.int(), kc, None)
    with pytest.raises(ValueError, match="fewer than cache_len"):
        rope_qk_cache_hip(q, k, None, cos[:16], sin[:16], pos, kc, None)
    with pytest.raises(ValueError, match="both"):
        rope_qk_cache_hip(q, k, k, cos, sin, pos, kc, None)


def test_rope_every_iteration_count() -> None:
    from ako_amd import _native

    x = grandn((3, 7, 40, 128), torch.float16, 14)
    cos, sin = build_rope_tables(7, 128, device=DEV)
    expected = oracle.rope(to_np(x), to_np(cos), to_np(sin), "neox", dtype="float16")
    try:
        for iters in (1, 2, 4, 8):
            _native.set_tuning(1, 2, iters)
            assert_rope_exact(expected, to_np(rope_hip(x, cos, sin)), torch.float16)
    finally:
        _native.set_tuning(1, 2, 0)


def test_rope_xcd_runs_cover_every_head() -> None:
    """RoPE with workgroups handed to the XCDs in runs (key 3; by default
    runs of 128 for one tensor from 8192 workgroups, as configs[2]'s q alone
    at (4, 2048) takes, checked against the oracle in test_rope_config3): the
    map is a bijection on the grid, so every run length, including ones that
    leave a partial last round and trailing blocks, gives the oracle's exact
    output, for q alone and for q and k in one launch."""
    from ako_amd import _native

    q = grandn((3, 37, 32, 128), torch.bfloat16, 15)
    k = grandn((3, 37, 8, 128), torch.bfloat16, 16)
    cos, sin = build_rope_tables(37, 128, device=DEV)
    cos, sin = cos.to(torch.bfloat16), sin.to(torch.bfloat16)
    eq = oracle.rope(to_np(q), to_np(cos), to_np(sin), "neox", dtype="bfloat16", table_dtype="bfloat16")
    ek = oracle.rope(to_np(k), to_np(cos), to_np(sin), "neox", dtype="bfloat16", table_dtype="bfloat16")
    try:
        for chunk in (0, 1, 2, 3, 8, 16, 1000):
            _native.set_tuning(1, 3, chunk)
            assert_rope_exact(eq, to_np(rope_hip(q, cos, sin)), torch.bfloat16)
            qo, ko = rope_qk_hip(q, k, cos, sin)
            assert_rope_exact(eq, to_np(qo), torch.bfloat16)
            assert_rope_exact(ek, to_np(ko), torch.bfloat16)
    finally:
        _native.set_tuning(1, 3, 0)


def test_rope_rejects_bad_input() -> None:
    x = torch.ones(1, 4, 2, 8, device=DEV, dtype=torch.float16)
    cos, sin = build_rope_tables(4, 8, device=DEV)
    with pytest.raises(ValueError):
        rope_hip(x, cos[:2], sin[:2])
    with pytest.raises(ValueError):
        rope_hip(x, cos, sin, "unknown-style")


# ------------------------------------------------------------------------ SwiGLU --


@pytest.mark.parametrize("m", [1, 16, 256, 4096, 16384])
def test_swiglu_config4(m: int) -> None:
    g = grandn((m, 14336), torch.bfloat16, 0)
    u = grandn((m, 14336), torch.bfloat16, 1)
    y = swiglu_hip(g, u)
    assert_gate(swiglu_ref(g, u), y)
    sel = torch.as_tensor(sample_rows(m, 512), device=DEV)
    assert_oracle(oracle.swiglu(to_np(g[sel]), to_np(u[sel]), dtype="bfloat16"), to_np(y[sel]),
                  torch.bfloat16)


@pytest.mark.parametrize("rows", [77, 300])
def test_swiglu_xcd_runs_cover_every_packet(rows: int) -> None:
    """Dense SwiGLU with workgroups handed to the XCDs in runs (key 2; by
    default runs of 4 for launches of 2048-65535 workgroups, which 300 rows
    of 14343 reach with 2101 and 77 rows do not): the map is a bijection on
    the grid, so every run length, including ones that leave a partial last
    round and trailing workgroups, gives the block-order output bit for bit,
    and the tail elements past the last full packet are still written."""
    from ako_amd import _native

    g = grandn((rows, 14343), torch.bfloat16, 17, scale=4.0)
    u = grandn((rows, 14343), torch.bfloat16, 18)
    try:
        _native.set_tuning(2, 2, 1)
        want = swiglu_hip(g, u)
        assert_oracle(oracle.swiglu(to_np(g), to_np(u), dtype="bfloat16"), to_np(want), torch.bfloat16)
        for chunk in (0, 2, 3, 4, 8, 64, 100000):
            _native.set_tuning(2, 2, chunk)
            assert torch.equal(swiglu_hip(g, u), want), chunk
    finally:
        _native.set_tuning(2, 2, 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(8, 2048, 5632), (2, 8448), (3, 1001), (1, 1), (7,), (4, 12)])
def test_swiglu_shapes(shape, dtype) -> None:
    g = grandn(shape, dtype, 15, scale=4.0)
    u = grandn(shape, dtype, 16)
    y = swiglu_hip(g, u)
    assert_gate(swiglu_ref(g, u), y)
    assert_oracle(oracle.swiglu(to_np(g), to_np(u), dtype=NAMES[dtype]), to_np(y), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_swiglu_extremes_and_strides(dtype) -> None:
    vals = torch.tensor([-100.0, -20.0, -5.0, -1.0, -0.0, 0.0, 1e-3, 1.0, 5.0, 20.0, 60.0], device=DEV)
    g = vals.repeat(64).reshape(8, -1).to(dtype)
    u = grandn(g.shape, dtype, 17)
    assert_oracle(oracle.swiglu(to_np(g), to_np(u), dtype=NAMES[dtype]), to_np(swiglu_hip(g, u)), dtype)
    base_g = grandn((16, 4096 + 8), dtype, 18)
    base_u = grandn((16, 4096 + 8), dtype, 19)
    gs, us = base_g[:, :4096], base_u[:, 8:]
    assert_oracle(oracle.swiglu(to_np(gs), to_np(us), dtype=NAMES[dtype]), to_np(swiglu_hip(gs, us)), dtype)
    gm = base_g.reshape(-1)[1:1 + 4096 * 3].view(3, 4096)  # misaligned: scalar path
    um = base_u.reshape(-1)[3:3 + 4096 * 3].view(3, 4096)
    assert_oracle(oracle.swiglu(to_np(gm), to_np(um), dtype=NAMES[dtype]), to_np(swiglu_hip(gm, um)), dtype)
    empty = torch.empty(0, 14336, device=DEV, dtype=dtype)
    assert swiglu_hip(empty, empty).shape == (0, 14336)


@pytest.mark.parametrize("binding", ["cpp", "ctypes"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_views_with_size1_leading_dims(dtype, binding) -> None:
    """4-D views whose leading dims cannot be walked with one row stride
    (a size-1 dim in front of a sliced one: rows 0..3 are 256 elements apart,
    row 4 is 2048 further) and views that can (a size-1 row dim whose rows
    sit at the outer stride). Each must give the contiguous input's result."""
    from ako_amd import _native
    from ako_amd.ops import rmsnorm_hip as rm
    from ako_amd.ops import swiglu_hip as sw

    fast = _native.torch_binding()
    if binding == "cpp":
        if fast is None:
            pytest.skip("the C++ binding is not built")
        f_rms, f_res, f_sw = fast.rmsnorm, fast.rmsnorm_residual, fast.swiglu
    else:
        f_rms, f_res, f_sw = rm.rmsnorm_hip_ctypes, rm.rmsnorm_residual_hip_ctypes, sw.swiglu_hip_ctypes
    h = 256
    big_x = grandn((2, 1, 8, h), dtype, 40)
    big_r = grandn((2, 1, 8, h), dtype, 41)
    w = grandn((h,), dtype, 42, scale=0.1, shift=1.0)
    views = [
        (big_x[:, :, :4, :], big_r[:, :, :4, :]),
        (big_x[:, :, 2:3, :], big_r[:, :, 5:6, :]),
        (big_x.permute(2, 1, 0, 3)[:3], big_r.permute(2, 1, 0, 3)[:3]),
    ]
    for x, r in views:
        xc, rc = x.contiguous(), r.contiguous()
        ey = oracle.rmsnorm(to_np(xc), to_np(w), dtype=NAMES[dtype])
        y = f_rms(x, w, 1e-6)
        assert y.shape == x.shape
        assert_oracle(ey, to_np(y), dtype)
        assert torch.equal(y, f_rms(xc, w, 1e-6))
        y2, s2 = f_res(x, r, w, 1e-6)
        ey2, es2 = oracle.rmsnorm_residual(to_np(xc), to_np(rc), to_np(w), dtype=NAMES[dtype])
        np.testing.assert_array_equal(to_np(s2), es2)
        assert_oracle(ey2, to_np(y2), dtype)
        g = f_sw(x, r)
        assert_oracle(oracle.swiglu(to_np(xc), to_np(rc), dtype=NAMES[dtype]), to_np(g), dtype)
        assert torch.equal(g, f_sw(xc, rc))


def _ordered16(bits: np.ndarray) -> np.ndarray:
    """16-bit float patterns mapped to integers in value order (+0 and -0 equal),
    so that the difference of two is their distance in ulps."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_swiglu_every_finite_half_gate(dtype) -> None:
    """silu(g) * u for every finite 16-bit gate value, with u = 1 and with
    seeded u, element by element within 1 ulp of the oracle (the fp32 math
    uses v_exp_f32 / v_rcp_f32 for half outputs). bf16 gates in
    [-88.7, -87.3] give normal fp32 results near 1e-37 whose reciprocal step
    would be subnormal; the kernel rescales there."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exp_mask, exp_all = (0x7C00, 0x7C00) if dtype == torch.float16 else (0x7F80, 0x7F80)
    bits = bits[(bits & exp_mask) != exp_all]  # finite values only
    g = torch.from_numpy(bits.view(np.int16).copy()).to(DEV).view(dtype)
    for u in (torch.ones_like(g), grandn(g.shape, dtype, 23)):
        y = swiglu_hip(g, u)
        ref = oracle.swiglu(to_np(g), to_np(u), dtype=NAMES[dtype])
        ref_bits = ref.view(np.uint16) if ref.dtype != np.uint16 else ref
        got_bits = y.view(torch.int16).cpu().numpy().view(np.uint16)
        dist = np.abs(_ordered16(got_bits) - _ordered16(ref_bits))
        worst = int(np.argmax(dist))
        assert dist.max() <= 1, (f"{dist.max()} ulp at gate {float(g[worst])} (bits {int(bits[worst]):#06x}): "
                                 f"got bits {int(got_bits[worst]):#06x}, oracle {int(ref_bits[worst]):#06x}; "
                                 f"{int((dist > 0).sum())} of {dist.size} differ")


def _finite16(dtype) -> np.ndarray:
    """Every finite 16-bit pattern of ``dtype`` (fp16 or bf16)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mask = 0x7C00 if dtype == torch.float16 else 0x7F80
    return bits[(bits & mask) != mask]


def _bits_tensor(bits: np.ndarray, dtype) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).to(DEV).view(dtype)


def _ulp_dist(got: torch.Tensor, ref: np.ndarray) -> np.ndarray:
    """Element-wise distance in ulps; two NaNs (of any sign or payload) are 0
    apart, a NaN and a number 65536."""
    got_bits = got.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    ref_bits = (ref.view(np.uint16) if ref.dtype != np.uint16 else ref).reshape(-1)
    exp_mask = 0x7C00 if got.dtype == torch.float16 else 0x7F80

    def nan(b: np.ndarray) -> np.ndarray:
        return ((b & exp_mask) == exp_mask) & ((b & ~np.uint16(0x8000 | exp_mask)) != 0)

    dist = np.abs(_ordered16(got_bits) - _ordered16(ref_bits))
    gn, rn = nan(got_bits), nan(ref_bits)
    return np.where(gn & rn, 0, np.where(gn ^ rn, 65536, dist))


@pytest.mark.parametrize("style", ["neox", "interleaved"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rope_every_finite_half_value(dtype, style) -> None:
    """Every finite 16-bit value as the first and as the second element of a
    rotated pair, at 255 positions with tables in the input dtype: the kernel
    rounds the same fp32 products and sums as the oracle, element by element
    within 1 ulp."""
    bits = _finite16(dtype)
    n = bits.size  # 63488 (fp16) or 65280 (bf16)
    heads = n // (255 * 128) if n % (255 * 128) == 0 else None
    rng = np.random.default_rng(31)
    cos, sin = build_rope_tables(256, 128, device=DEV)
    cos, sin = cos.to(dtype), sin.to(dtype)
    for perm in (np.arange(n), rng.permutation(n)):
        flat = bits[perm]
        pad = (-flat.size) % (256 * 128)
        flat = np.concatenate([flat, np.zeros(pad, dtype=np.uint16)])
        x = _bits_tensor(flat, dtype).view(1, 256, -1, 128)
        y = rope_hip(x, cos, sin, style)
        ref = oracle.rope(to_np(x), to_np(cos), to_np(sin), style, dtype=NAMES[dtype], table_dtype=NAMES[dtype])
        dist = _ulp_dist(y, ref)
        assert dist.max() <= 1, f"{dist.max()} ulp; {int((dist > 0).sum())} of {dist.size} differ"
    assert heads is None or heads >= 1


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("copies", [1, 1821], ids=["9rows", "16389rows"])
def test_rmsnorm_extreme_rows(dtype, copies) -> None:
    """Rows of subnormals, rows near the format's maximum (whose sum of squares
    overflows fp32 for bf16), a single non-zero element, zeros, and mixes,
    plain and residual: element by element within 1 ulp of the oracle (the
    rounded residual sum exactly). The nine rows run as one launch of nine
    (the register kernel) and repeated 1821 times, which the persistent
    pipelined kernel takes."""
    rng = np.random.default_rng(37)
    h = 4096
    if dtype == torch.float16:
        sub, big = (0x0001, 0x03FF), (0x7800, 0x7BFF)   # subnormals; 32768 .. 65504
    else:
        sub, big = (0x0001, 0x007F), (0x7E00, 0x7F7F)   # subnormals; 4.3e37 .. 3.4e38
    rows = []
    for lo, hi in (sub, big):
        for sign in (0, 0x8000):
            rows.append(rng.integers(lo, hi + 1, h, dtype=np.uint32).astype(np.uint16) | np.uint16(sign))
    one = np.zeros(h, dtype=np.uint16)
    one[rng.integers(h)] = 0x3C00 if dtype == torch.float16 else 0x3F80  # a single 1.0
    rows += [one, np.zeros(h, dtype=np.uint16)]
    mix = rng.integers(sub[0], sub[1] + 1, h, dtype=np.uint32).astype(np.uint16)
    mix[::97] = rng.integers(big[0], big[1] + 1, mix[::97].size, dtype=np.uint32).astype(np.uint16)
    rows.append(mix)
    x = _bits_tensor(np.stack(rows), dtype)
    r = _bits_tensor(np.stack(rows[::-1]), dtype)
    w = grandn((h,), dtype, 41, scale=0.1, shift=1.0)
    big_x, big_r = x.repeat(copies, 1), r.repeat(copies, 1)

    def tiled(a: np.ndarray) -> np.ndarray:
        return np.tile(a, (copies, 1))

    for eps in (1e-6, 0.0):
        y = rmsnorm_hip(big_x, w, eps)
        dist = _ulp_dist(y, tiled(oracle.rmsnorm(to_np(x), to_np(w), eps, dtype=NAMES[dtype])))
        assert dist.max() <= 1, f"plain eps={eps}: {dist.max()} ulp; {int((dist > 0).sum())} differ"
        y, s = rmsnorm_residual_hip(big_x, big_r, w, eps)
        ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), eps, dtype=NAMES[dtype])
        ey, es = tiled(ey), tiled(es)
        assert _ulp_dist(s, es).max() == 0
        dist = _ulp_dist(y, ey)
        assert dist.max() <= 1, f"residual eps={eps}: {dist.max()} ulp; {int((dist > 0).sum())} differ"


def _with_specials(shape, dtype, seed: int, hits: list[tuple[tuple, float]]) -> torch.Tensor:
    """Seeded N(0,1) values with the given (index, value) entries overwritten."""
    t = grandn(shape, torch.float32, seed)
    for idx, val in hits:
        t[idx] = val
    return t.to(dtype)


@pytest.mark.parametrize("copies", [1, 1100], ids=["16rows", "17600rows"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_nonfinite_inputs_propagate_like_the_oracle(dtype, copies) -> None:
    """NaN and infinities in the inputs: every kernel gives the oracle's
    results, NaN where the oracle has NaN (any payload) and the same numbers
    elsewhere (RMSNorm and SwiGLU within 1 ulp, RoPE exactly). A row holding
    an infinity has an infinite sum of squares, so its finite elements
    normalise to 0 and the infinity to NaN (inf * 0), as in the unfused
    reference. RMSNorm runs both as 16 rows (the register kernel) and
    repeated 1100 times (17600 rows: the pipelined kernel; bf16 residual rows
    of this width keep the register kernel)."""
    inf, nan = float("inf"), float("nan")
    h = 4096
    x = _with_specials((16, h), dtype, 70, [((0, 5), inf), ((1, 9), -inf), ((2, 100), nan), ((3, 1), inf),
                                             ((3, 2), -inf), ((7, 300), inf), ((9, 0), nan), ((9, 1), inf)])
    r = _with_specials((16, h), dtype, 71, [((5, 17), inf), ((6, 33), nan), ((7, 300), -inf), ((8, 4), -inf)])
    w = grandn((h,), dtype, 72, scale=0.1, shift=1.0)
    bx, br = x.repeat(copies, 1), r.repeat(copies, 1)

    def tiled(a):
        return np.tile(a, (copies, 1))

    dist = _ulp_dist(rmsnorm_hip(bx, w), tiled(oracle.rmsnorm(to_np(x), to_np(w), dtype=NAMES[dtype])))
    assert dist.max() <= 1, f"rmsnorm: {dist.max()} ulp; {int((dist > 0).sum())} differ"
    y, s_ = rmsnorm_residual_hip(bx, br, w)
    ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), dtype=NAMES[dtype])
    assert _ulp_dist(s_, tiled(es)).max() == 0
    dist = _ulp_dist(y, tiled(ey))
    assert dist.max() <= 1, f"rmsnorm_residual: {dist.max()} ulp; {int((dist > 0).sum())} differ"
    if copies > 1:
        return
    q = _with_specials((2, 8, 4, 128), dtype, 73, [((0, 1, 0, 3), inf), ((0, 2, 1, 70), -inf), ((1, 3, 2, 0), nan),
                                                   ((1, 7, 3, 64), inf), ((1, 7, 3, 0), nan)])
    cos, sin = build_rope_tables(8, 128, device=DEV)
    cos, sin = cos.to(dtype), sin.to(dtype)
    for style in ("neox", "interleaved"):
        dist = _ulp_dist(rope_hip(q, cos, sin, style),
                         oracle.rope(to_np(q), to_np(cos), to_np(sin), style, dtype=NAMES[dtype],
                                     table_dtype=NAMES[dtype]))
        assert dist.max() == 0, f"rope {style}: {dist.max()} ulp; {int((dist > 0).sum())} differ"
    g = _with_specials((64, h), dtype, 74, [((0, 0), inf), ((1, 1), -inf), ((2, 2), nan), ((3, 3), 0.0),
                                             ((4, 4), 1.0)])
    u = _with_specials((64, h), dtype, 75, [((3, 3), inf), ((4, 4), -inf), ((5, 5), nan), ((6, 6), inf)])
    dist = _ulp_dist(swiglu_hip(g, u), oracle.swiglu(to_np(g), to_np(u), dtype=NAMES[dtype]))
    assert dist.max() <= 1, f"swiglu: {dist.max()} ulp; {int((dist > 0).sum())} differ"


def _ordered32(a: np.ndarray) -> np.ndarray:
    b = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.int64)
    return np.where(b & 0x80000000, 0x80000000 - (b & 0x7FFFFFFF), 0x80000000 + b)


def _ulp_dist32(got: np.ndarray, ref: np.ndarray) -> np.ndarray:
    got, ref = np.asarray(got, np.float32).reshape(-1), np.asarray(ref, np.float32).reshape(-1)
    dist = np.abs(_ordered32(got) - _ordered32(ref))
    gn, rn = np.isnan(got), np.isnan(ref)
    return np.where(gn & rn, 0, np.where(gn ^ rn, 1 << 32, dist))


def test_fp32_extremes_element_by_element() -> None:
    """fp32 RMSNorm (rows of subnormals, of values near 1e38 whose squares
    overflow, a single non-zero element, zeros) and fp32 SwiGLU over gates
    from -100 to 100 including subnormals: within 4 ulp of the oracle element
    by element (the fp32 target)."""
    rng = np.random.default_rng(43)
    h = 4096
    rows = [
        rng.uniform(1e-41, 1e-39, h) * rng.choice([-1, 1], h),  # subnormal
        rng.uniform(1e37, 3e38, h) * rng.choice([-1, 1], h),    # squares overflow
        np.zeros(h),
        rng.standard_normal(h) * 1e-20,
    ]
    one = np.zeros(h)
    one[rng.integers(h)] = 1.0
    rows.append(one)
    x = torch.tensor(np.stack(rows), dtype=torch.float32, device=DEV)
    w = grandn((h,), torch.float32, 47, scale=0.1, shift=1.0)
    for eps in (1e-6, 0.0):
        ref = oracle.rmsnorm(to_np(x), to_np(w), eps, dtype="float32")
        dist = _ulp_dist32(to_np(rmsnorm_hip(x, w, eps)), ref)
        assert dist.max() <= 4, f"rmsnorm eps={eps}: {dist.max()} ulp"
    g = torch.tensor(np.concatenate([np.linspace(-100, 100, 200001), [1e-40, -1e-40, 0.0, -0.0, 1e-30]]),
                     dtype=torch.float32, device=DEV)
    u = grandn(g.shape, torch.float32, 53)
    ref = oracle.swiglu(to_np(g), to_np(u), dtype="float32")
    dist = _ulp_dist32(to_np(swiglu_hip(g, u)), ref)
    assert dist.max() <= 4, f"swiglu: {dist.max()} ulp at g={float(g[int(np.argmax(dist))])}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_element_by_element_at_config_shapes(dtype) -> None:
    """Element-wise distance to the oracle, which is tighter than the gate's
    max|ref|-relative budget. Half precision: at most 1 ulp for RMSNorm and
    SwiGLU, RoPE bit-exact. fp32: RMSNorm within 4 ulp (a different summation
    order moves rstd by a few ulp), RoPE bit-exact, SwiGLU within 4 ulp
    (the device's 1-ulp expf against the oracle's correctly rounded exp)."""
    half = dtype != torch.float32

    def dist(y, ref):
        return _ulp_dist(y, ref) if half else _ulp_dist32(to_np(y), ref)

    for rows, h in ((1, 4096), (32, 8192), (16384, 16384)):
        x, r = grandn((rows, h), dtype, 0), grandn((rows, h), dtype, 2)
        w = grandn((h,), dtype, 1, scale=0.1, shift=1.0)
        sel = torch.as_tensor(sample_rows(rows), device=DEV)
        d = dist(rmsnorm_hip(x, w, 1e-6)[sel], oracle.rmsnorm(to_np(x[sel]), to_np(w), 1e-6, dtype=NAMES[dtype]))
        assert d.max() <= (1 if half else 4), (rows, h, int(d.max()))
        y, s = rmsnorm_residual_hip(x, r, w, 1e-6)
        ey, es = oracle.rmsnorm_residual(to_np(x[sel]), to_np(r[sel]), to_np(w), 1e-6, dtype=NAMES[dtype])
        assert dist(s[sel], es).max() == 0
        assert dist(y[sel], ey).max() <= (1 if half else 4), (rows, h)
    cos, sin = build_rope_tables(2048, 128, device=DEV)
    for tdt in {torch.float32, dtype}:
        q = grandn((2, 2048, 32, 128), dtype, 5)
        ref = oracle.rope(to_np(q), to_np(cos.to(tdt)), to_np(sin.to(tdt)), dtype=NAMES[dtype], table_dtype=NAMES[tdt])
        assert dist(rope_hip(q, cos.to(tdt), sin.to(tdt)), ref).max() == 0
    g, u = grandn((512, 14336), dtype, 7, scale=3.0), grandn((512, 14336), dtype, 8)
    d = dist(swiglu_hip(g, u), oracle.swiglu(to_np(g), to_np(u), dtype=NAMES[dtype]))
    assert d.max() <= (1 if half else 4), int(d.max())


def test_tensors_beyond_2_31_elements() -> None:
    """Each kernel on a tensor of more than 2^31 elements (over 4 GiB in
    fp16), so element offsets need 64 bits: the last rows / tokens and a
    seeded sample against the oracle (RoPE bit for bit, the residual sum
    exactly, the rest within 1 ulp element by element)."""
    rng = np.random.default_rng(71)

    def pick(n: int) -> torch.Tensor:
        idx = np.unique(np.concatenate([[0, n - 3, n - 2, n - 1], rng.choice(n, 40, replace=False)]))
        return torch.as_tensor(idx, device=DEV)

    rows = (1 << 31) // 8192 + 3
    x, r = grandn((rows, 8192), torch.float16, 70), grandn((rows, 8192), torch.float16, 72)
    w = grandn((8192,), torch.float16, 74, scale=0.1, shift=1.0)
    assert x.numel() > (1 << 31)
    y, s = rmsnorm_residual_hip(x, r, w, 1e-6)
    sel = pick(rows)
    ey, es = oracle.rmsnorm_residual(to_np(x[sel]), to_np(r[sel]), to_np(w), 1e-6, dtype="float16")
    np.testing.assert_array_equal(to_np(s[sel]), es)
    assert _ulp_dist(y[sel], ey).max() <= 1
    del r, y, s
    # Plain rows of 8192 here take the persistent pipelined kernel.
    y = rmsnorm_hip(x, w, 1e-6)
    assert _ulp_dist(y[sel], oracle.rmsnorm(to_np(x[sel]), to_np(w), 1e-6, dtype="float16")).max() <= 1
    del x, y
    torch.cuda.empty_cache()

    # bf16 residual rows of 16384: one-packet load groups.
    rows = (1 << 31) // 16384 + 3
    x, r = grandn((rows, 16384), torch.bfloat16, 82), grandn((rows, 16384), torch.bfloat16, 84)
    w = grandn((16384,), torch.bfloat16, 86, scale=0.1, shift=1.0)
    y, s = rmsnorm_residual_hip(x, r, w, 1e-6)
    sel = pick(rows)
    ey, es = oracle.rmsnorm_residual(to_np(x[sel]), to_np(r[sel]), to_np(w), 1e-6, dtype="bfloat16")
    np.testing.assert_array_equal(to_np(s[sel]), es)
    assert _ulp_dist(y[sel], ey).max() <= 1
    del x, r, y, s
    torch.cuda.empty_cache()

    m = (1 << 31) // 14336 + 2
    g, u = grandn((m, 14336), torch.bfloat16, 76), grandn((m, 14336), torch.bfloat16, 78)
    y = swiglu_hip(g, u)
    sel = pick(m)
    assert _ulp_dist(y[sel], oracle.swiglu(to_np(g[sel]), to_np(u[sel]), dtype="bfloat16")).max() <= 1
    del g, u, y
    torch.cuda.empty_cache()

    seq = (1 << 31) // (128 * 128) + 2
    x = grandn((1, seq, 128, 128), torch.float16, 80)
    cos, sin = build_rope_tables(seq, 128, device=DEV)
    y = rope_hip(x, cos, sin)
    sel = pick(seq)
    expected = oracle.rope(to_np(x[:, sel]), to_np(cos[sel]), to_np(sin[sel]), "neox", dtype="float16")
    np.testing.assert_array_equal(to_np(y[:, sel]), expected)
    del x, y
    torch.cuda.empty_cache()


def _bf16_pairs() -> tuple[np.ndarray, np.ndarray]:
    """Every bf16 pattern (x) against eight partners (r): two random
    permutations, itself (doubling: overflow, subnormals doubled), its
    negation (exact cancellation to +0, -0 + +0), +0, -0, and the smallest
    positive and negative subnormals (steps across zero and the subnormal
    range). 524288 pairs."""
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(91)
    partners = [rng.permutation(every), rng.permutation(every), every, every ^ np.uint16(0x8000),
                np.zeros_like(every), np.full_like(every, 0x8000), np.full_like(every, 0x0001),
                np.full_like(every, 0x8001)]
    return np.tile(every, len(partners)), np.concatenate(partners)


def _assert_same_bits(got: torch.Tensor, ref_bits: np.ndarray, what: str) -> None:
    """Bit-identical, except that two NaNs match whatever their payloads."""
    g = got.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    r = ref_bits.reshape(-1)

    def nan(b):
        return ((b & 0x7F80) == 0x7F80) & ((b & 0x007F) != 0)

    bad = (g != r) & ~(nan(g) & nan(r))
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} differ, first at {int(np.argmax(bad))}: "
                           f"got {g[bad][:4]}, want {r[bad][:4]}")


# (hidden, rows of the 524288 pairs repeated `copies` times): the residual
# sum through each kernel that adds packets: rmsnorm_reg at (8, 1) with early
# weights and through rmsnorm_pipe (4096), at (16, 1) (8192), at (16, 2)
# (16384; from 257 rows with write-through stores and one packet per load
# group), and
# rmsnorm_stream for rows past the register budget (131072).
BF16_SUM_CASES = [(4096, 1), (4096, 3), (8192, 1), (8192, 5), (16384, 1), (16384, 9), (131072, 1)]


@pytest.mark.parametrize("hidden,copies", BF16_SUM_CASES, ids=[f"{h}x{c}" for h, c in BF16_SUM_CASES])
def test_bf16_residual_sum_every_pattern(hidden, copies) -> None:
    """The rounded residual sum s = bf16(x + r) for every bf16 x against
    eight partners each (signed zeros, subnormals, overflow to infinity,
    cancellation, NaN and infinities included), bit for bit against the
    oracle's fp32 add and round-to-nearest-even, through every kernel that
    adds 16-byte packets. The tensor-parallel partial half, which adds the
    same way, is checked on the same pairs."""
    from ako_amd.ops.rmsnorm_tp import rmsnorm_shard_partial_hip

    xb, rb = _bf16_pairs()
    with np.errstate(over="ignore", invalid="ignore"):  # overflow to inf and inf - inf are among the cases
        want = oracle.round_to(oracle.to_f32(xb, "bfloat16") + oracle.to_f32(rb, "bfloat16"), "bfloat16")
    x = _bits_tensor(xb.reshape(-1, hidden), torch.bfloat16).repeat(copies, 1)
    r = _bits_tensor(rb.reshape(-1, hidden), torch.bfloat16).repeat(copies, 1)
    w = torch.ones(hidden, dtype=torch.bfloat16, device=DEV)
    _, s = rmsnorm_residual_hip(x, r, w)
    _assert_same_bits(s, np.tile(want.reshape(-1, hidden), (copies, 1)), f"rmsnorm_residual {tuple(x.shape)}")
    if copies == 1 and hidden <= 8192:
        s_tp, _ = rmsnorm_shard_partial_hip(x, r)
        _assert_same_bits(s_tp, want, f"rmsnorm_shard_partial {tuple(x.shape)}")
