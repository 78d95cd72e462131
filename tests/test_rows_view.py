"""Row-walk of strided inputs (``rows_view``), checked on the CPU by brute force.

A kernel reads row ``r`` of the last dimension at ``r * row_stride``. Whenever
``rows_view`` hands a tensor through without a copy, that formula must give the
storage offset of every row, which is checked here against torch's own indexing
for each leading index. The planted case (a size-1 dim in front of a sliced dim
of a 4-D view) is the one a check that compared neighbouring dims only got
wrong: it returned row stride 8 for rows that sit 64 apart.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from ako_amd.ops._hip_common import leading_row_stride, rows_view


def row_offsets(t: torch.Tensor) -> list[int]:
    """Storage offset of element 0 of every row, in row-major order."""
    base = t.storage_offset()
    out = []
    for idx in itertools.product(*(range(s) for s in t.shape[:-1])):
        out.append(t[idx].storage_offset() - base if t.shape[-1] else 0)
    return out


def check_walk(t: torch.Tensor) -> bool:
    """True when rows_view avoided a copy; asserts the walk is right either way."""
    v, stride = rows_view(t)
    rows = int(np.prod(t.shape[:-1])) if t.dim() > 1 else 1
    if v.data_ptr() != t.data_ptr():
        assert v.is_contiguous() and stride == t.shape[-1]
        torch.testing.assert_close(v, t, rtol=0, atol=0)
        return False
    offs = row_offsets(t)
    assert offs == [r * stride for r in range(rows)], (tuple(t.shape), t.stride(), stride)
    if rows > 1:
        assert stride >= t.shape[-1]
    return True


def test_size1_dim_before_a_sliced_dim():
    big = torch.arange(2 * 1 * 8 * 8, dtype=torch.float32).view(2, 1, 8, 8)
    x = big[:, :, :4, :]
    assert x.stride() == (64, 64, 8, 1)
    # Rows of x do not sit at one stride (0, 8, 16, 24, then 64 ...): copy.
    assert leading_row_stride(tuple(x.shape), x.stride()) is None
    assert not check_walk(x)
    # Take the full dim 2 instead: rows are every 8 elements, no copy.
    assert check_walk(big[:, :, :, :])
    # A non-contiguous view whose rows do sit at one stride: padded last dim.
    padded = torch.zeros(3, 1, 5, 12)[..., :10]
    assert check_walk(padded)
    assert rows_view(padded)[1] == 12


def test_size1_row_dim_uses_the_outer_stride():
    base = torch.zeros(4, 3, 16)
    x = base[:, 1:2, :8]                       # shape (4,1,8), strides (48,16,1)
    v, stride = rows_view(x)
    assert v.data_ptr() == x.data_ptr() and stride == 48
    assert check_walk(x)


def test_expanded_rows_are_copied():
    x = torch.randn(1, 8).expand(5, 8)         # row stride 0 overlaps rows
    assert not check_walk(x)


@pytest.mark.parametrize("seed", range(40))
def test_random_views_walk_correctly(seed):
    rng = np.random.default_rng(seed)
    nd = int(rng.integers(2, 6))
    shape = [int(rng.integers(1, 5)) for _ in range(nd)]
    shape[-1] = int(rng.integers(1, 9))
    big = torch.arange(int(np.prod([s + 2 for s in shape])), dtype=torch.float32).view(
        *[s + 2 for s in shape])
    # Random slices (some full, some short, some of length 1), then maybe a
    # permutation of the leading dims.
    sl = []
    for s in shape:
        start = int(rng.integers(0, 3))
        sl.append(slice(start, start + s))
    x = big[tuple(sl)]
    if rng.random() < 0.4 and nd > 2:
        perm = list(rng.permutation(nd - 1)) + [nd - 1]
        x = x.permute(*perm)
    if rng.random() < 0.3:
        x = x.unsqueeze(int(rng.integers(0, x.dim())))
    check_walk(x)


def _binding():
    from ako_amd import _native

    try:
        return _native.torch_binding()
    except Exception:  # noqa: BLE001 - an unbuilt binding just skips
        return None


@pytest.mark.parametrize("seed", range(40))
def test_cpp_binding_walks_like_python(seed):
    """The C++ binding's copy of the walk gives the same decision and stride."""
    fast = _binding()
    if fast is None or not hasattr(fast, "row_walk"):
        pytest.skip("the C++ binding is not built")
    rng = np.random.default_rng(1000 + seed)
    nd = int(rng.integers(2, 6))
    shape = [int(rng.integers(1, 4)) for _ in range(nd)]
    big = torch.zeros(*[s + 2 for s in shape])
    x = big[tuple(slice(int(rng.integers(0, 3)), None) for _ in shape)]
    x = x[tuple(slice(0, s) for s in shape)]
    if rng.random() < 0.4 and nd > 2:
        x = x.permute(*(list(rng.permutation(nd - 1)) + [nd - 1]))
    v, stride = rows_view(x)
    copied, cstride = fast.row_walk(x)
    assert copied == (v.data_ptr() != x.data_ptr())
    assert cstride == stride


def test_cpp_binding_planted_case():
    fast = _binding()
    if fast is None or not hasattr(fast, "row_walk"):
        pytest.skip("the C++ binding is not built")
    big = torch.zeros(2, 1, 8, 8)
    assert fast.row_walk(big[:, :, :4, :]) == (True, 8)
    assert fast.row_walk(torch.zeros(4, 3, 16)[:, 1:2, :8]) == (False, 48)
