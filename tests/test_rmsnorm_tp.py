"""RMSNorm over a hidden dimension split into tensor-parallel slices.

CPU: the PyTorch halves compose to the full-row reference and to the oracle,
and the C ABI validates its arguments. GPU (marked): the HIP halves at the
configs[1] shapes, every slice count, plain and residual, against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ako_amd import _native
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref, rmsnorm_residual_ref
from ako_amd.ops.rmsnorm_tp import (
    rmsnorm_shard_apply_hip,
    rmsnorm_shard_apply_ref,
    rmsnorm_shard_partial_hip,
    rmsnorm_shard_partial_ref,
    rmsnorm_sharded,
)
from ako_amd.validation.numerical import error_budget, max_abs_error
from oracle import ops as oracle
from tests._util import NAMES, randn, to_np

REFS = dict(partial_fn=rmsnorm_shard_partial_ref, apply_fn=rmsnorm_shard_apply_ref)


def drandn(shape, dtype, seed, *, scale=1.0, shift=0.0) -> torch.Tensor:
    """Seeded normal values drawn on the GPU (full-size configs[1] inputs)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, generator=g, device="cuda") * scale + shift).to(dtype)
MAX_ULPS = 2.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shards", [1, 2, 4, 8])
def test_reference_slices_compose_to_the_full_row(dtype: torch.dtype, shards: int) -> None:
    x, r = randn((6, 512), dtype, 1), randn((6, 512), dtype, 2)
    w = randn((512,), dtype, 3, scale=0.1, shift=1.0)
    y, s = rmsnorm_sharded(x, r, w, 1e-6, shards=shards, **REFS)
    ey, es = rmsnorm_residual_ref(x, r, w, 1e-6)
    assert torch.equal(s, es)  # the residual sum is elementwise: identical
    assert max_abs_error(ey, y) <= error_budget(ey)
    rep = oracle.gate(oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), dtype=NAMES[dtype])[0],
                      to_np(y), NAMES[dtype])
    assert rep["passed"] and rep["err_ulps"] <= MAX_ULPS, rep
    yp, sp = rmsnorm_sharded(x, None, w, 1e-6, shards=shards, **REFS)
    assert sp is not None and torch.equal(sp, x)
    assert max_abs_error(rmsnorm_ref(x, w, 1e-6), yp) <= error_budget(yp)
    with pytest.raises(ValueError, match="divisible"):
        rmsnorm_sharded(x, r, w, shards=3, **REFS)


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="passes fake device addresses: runs only where no GPU is visible")
def test_shard_abi_validation() -> None:
    lib = _native.load()
    A, B, C, D = 0x100000, 0x200000, 0x300000, 0x400000
    p = lib.ako_rmsnorm_shard_partial_fwd
    assert p(A, None, None, D, 0, 64, 64, 0, 0, 1, None) == 0  # no rows: nothing to do
    assert p(A, B, None, D, 4, 64, 64, 64, 64, 1, None) == 1 and "both" in _native.last_error()
    assert p(A, None, None, None, 4, 64, 64, 0, 0, 1, None) == 1
    assert p(A, B, C, A + 8, 4, 64, 64, 64, 64, 1, None) == 1 and "overlaps" in _native.last_error()
    assert p(A, B, C, D, 4, 64, 64, 64, 32, 1, None) == 1 and "stride" in _native.last_error()
    assert p(A, None, None, D, 4, 64, 64, 0, 0, 9, None) == 2
    a = lib.ako_rmsnorm_shard_apply_fwd
    assert a(A, B, C, D, 4, 64, 32, 64, 64, 1e-6, 1, 1, None) == 1 and "larger than hidden" in _native.last_error()
    assert a(A, B, C, A, 4, 64, 128, 64, 64, 1e-6, 1, 1, None) == 1 and "overlaps" in _native.last_error()
    assert a(A, B, C, D, 4, 64, 128, 64, 64, -1.0, 1, 1, None) == 1
    assert a(A, B, C, D, 4, 64, 128, 64, 64, 1e-6, 1, 2, None) == 2
    assert a(A, B, C, D, 0, 64, 128, 64, 64, 1e-6, 1, 1, None) == 0




@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden,shards", [
    (rows, hidden, shards)
    for rows, hidden in [(1, 4096), (33, 16384), (16384, 16384), (4097, 2048), (5, 4100)]
    for shards in (1, 2, 8) if hidden % shards == 0
])
def test_hip_slices_compose_to_the_full_row(rows: int, hidden: int, shards: int, dtype) -> None:
    """configs[1] rows and widths cut into 1, 2 or 8 slices (TP=8 puts 2048 of
    16384 on a rank); 4097 rows leave the apply kernel's last workgroup (two
    rows each from 4096 rows on) one row; 4100/2 slices are not 16-byte
    aligned (scalar path)."""
    dev = "cuda"
    x, r = drandn((rows, hidden), dtype, 4), drandn((rows, hidden), dtype, 5)
    w = drandn((hidden,), dtype, 6, scale=0.1, shift=1.0)
    y, s = rmsnorm_sharded(x, r, w, 1e-6, shards=shards)
    sel = torch.as_tensor(np.unique(np.linspace(0, rows - 1, min(rows, 256)).astype(np.int64)), device=dev)
    ey, es = oracle.rmsnorm_residual(to_np(x[sel]), to_np(r[sel]), to_np(w), 1e-6, dtype=NAMES[dtype])
    np.testing.assert_array_equal(to_np(s[sel]), es)
    rep = oracle.gate(ey, to_np(y[sel]), NAMES[dtype])
    assert rep["passed"] and rep["err_ulps"] <= MAX_ULPS, rep
    yp, _ = rmsnorm_sharded(x, None, w, 1e-6, shards=shards)
    rep = oracle.gate(oracle.rmsnorm(to_np(x[sel]), to_np(w), 1e-6, dtype=NAMES[dtype]), to_np(yp[sel]),
                      NAMES[dtype])
    assert rep["passed"] and rep["err_ulps"] <= MAX_ULPS, rep


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_hip_partial_sums_and_weights() -> None:
    """The partial sums against float64, and an fp32 weight on half inputs."""
    dev = "cuda"
    x = randn((64, 2048), torch.bfloat16, 7, device=dev)
    r = randn((64, 2048), torch.bfloat16, 8, device=dev)
    s, part = rmsnorm_shard_partial_hip(x, r)
    s64 = (x.double() + r.double()).to(torch.bfloat16).double()
    torch.testing.assert_close(part.double(), s64.pow(2).sum(-1), rtol=1e-5, atol=0)
    _, part_x = rmsnorm_shard_partial_hip(x)
    torch.testing.assert_close(part_x.double(), x.double().pow(2).sum(-1), rtol=1e-5, atol=0)
    w32 = randn((2048,), torch.float32, 9, scale=0.1, shift=1.0, device=dev)
    y = rmsnorm_shard_apply_hip(s, w32, part, 2048, 1e-6)
    expected = oracle.rmsnorm(to_np(s), to_np(w32), 1e-6, dtype="bfloat16", w_dtype="float32")
    rep = oracle.gate(expected, to_np(y), "bfloat16")
    assert rep["passed"] and rep["err_ulps"] <= MAX_ULPS, rep
    with pytest.raises(ValueError, match="float32"):
        rmsnorm_shard_apply_hip(s, w32, part.double(), 2048)


def _free_port() -> int:
    import socket

    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _run_ranks(tmp_path, world: int, device: str, dtype: torch.dtype, rows: int, hidden: int,
               use_hip: bool) -> None:
    """Spawn ``world`` ranks over gloo; check the concatenated slices against
    the full-row reference (bit-equal residual sum, normalised rows within the
    gate and 2 ulps of the oracle)."""
    import torch.multiprocessing as mp

    from tests._tp_worker import full_inputs, rank_main

    mp.spawn(rank_main, args=(world, _free_port(), str(tmp_path), device, str(dtype).split(".")[-1], rows,
                              hidden, use_hip), nprocs=world, join=True)
    parts = [torch.load(tmp_path / f"rank{i}.pt", weights_only=True) for i in range(world)]
    y = torch.cat([p["y"] for p in parts], -1)
    s = torch.cat([p["s"] for p in parts], -1)
    yp = torch.cat([p["y_plain"] for p in parts], -1)
    x, r, w = full_inputs(rows, hidden, dtype)
    ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), 1e-6, dtype=NAMES[dtype])
    np.testing.assert_array_equal(to_np(s), es)
    rep = oracle.gate(ey, to_np(y), NAMES[dtype])
    assert rep["passed"] and rep["err_ulps"] <= MAX_ULPS, rep
    rep = oracle.gate(oracle.rmsnorm(to_np(x), to_np(w), 1e-6, dtype=NAMES[dtype]), to_np(yp), NAMES[dtype])
    assert rep["passed"] and rep["err_ulps"] <= MAX_ULPS, rep


def test_two_gloo_ranks_compose_to_the_full_row(tmp_path) -> None:
    """Two processes, each holding half of every row, all-reduce their partial
    sums over gloo (the PyTorch halves on the CPU)."""
    _run_ranks(tmp_path, 2, "cpu", torch.bfloat16, 16, 1024, use_hip=False)


def test_rank_rejects_a_mismatched_weight_slice() -> None:
    from ako_amd.ops.rmsnorm_tp import rmsnorm_tp

    x = torch.zeros(2, 8)
    with pytest.raises(ValueError, match="weight slice"):
        rmsnorm_tp(x, None, torch.ones(16), 16, partial_fn=rmsnorm_shard_partial_ref,
                   apply_fn=rmsnorm_shard_apply_ref)


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_two_ranks_on_the_gpu_compose_to_the_full_row(tmp_path, dtype) -> None:
    """The HIP halves in two processes sharing cuda:0; the partial sums cross
    gloo through host copies (4096 rows x 8192, each rank a 4096-wide slice)."""
    _run_ranks(tmp_path, 2, "cuda:0", dtype, 4096, 8192, use_hip=True)


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_hip_slices_extreme_rows() -> None:
    """Rows of subnormals, of values whose squares overflow fp32, zeros and a
    single non-zero element, cut into 4 slices: the composed result equals the
    full-row oracle element by element within 1 ulp, NaN where it is NaN."""
    from tests.test_hip_parity import _ulp_dist

    rng = np.random.default_rng(59)
    h = 4096
    rows = [rng.integers(0x0001, 0x0080, h, dtype=np.uint32).astype(np.uint16),
            rng.integers(0x7E00, 0x7F80, h, dtype=np.uint32).astype(np.uint16) | np.uint16(0x8000),
            np.zeros(h, dtype=np.uint16)]
    one = np.zeros(h, dtype=np.uint16)
    one[rng.integers(h)] = 0x3F80
    rows.append(one)
    bits = np.stack(rows)
    x = torch.from_numpy(bits.view(np.int16).copy()).cuda().view(torch.bfloat16)
    r = torch.from_numpy(bits[::-1].copy().view(np.int16)).cuda().view(torch.bfloat16)
    w = drandn((h,), torch.bfloat16, 61, scale=0.1, shift=1.0)
    y, s = rmsnorm_sharded(x, r, w, 1e-6, shards=4)
    ey, es = oracle.rmsnorm_residual(to_np(x), to_np(r), to_np(w), 1e-6, dtype="bfloat16")
    assert _ulp_dist(s, es).max() == 0
    assert _ulp_dist(y, ey).max() <= 1
