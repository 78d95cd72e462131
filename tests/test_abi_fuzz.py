"""Property test of the C ABI's host-side validation (no GPU, fake addresses).

For random argument sets, the library's answer is compared with the contract
in ``include/ako_hip.h``, stated here independently:

* sizes are non-negative; an empty problem is accepted before anything else;
* the width must fit in 31 bits; pointers must not be null; eps must be >= 0;
* row strides are non-negative, and an output's rows must not overlap
  (stride >= width when there is more than one row);
* no output byte range may overlap an input's, or the other output's.

A call the contract rejects must come back ``AKO_ERR_INVALID_ARGUMENT`` (1);
a call it accepts reaches the launch, which on a machine without a GPU reports
``AKO_ERR_NO_DEVICE`` (4). Never a crash, never a silent acceptance of an
overlap. The addresses are fake, so this module runs only where no GPU is
visible (a validation slip must not launch a kernel on them).
"""

from __future__ import annotations

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from ako_amd import _native

pytestmark = pytest.mark.skipif(torch.cuda.is_available(),
                                reason="passes fake device addresses: runs only where no GPU is visible")

INVALID, NO_DEVICE = 1, 4
EB = {0: 4, 1: 2, 2: 2}  # element bytes per dtype code


def byte_range(ptr: int, rows: int, width: int, stride: int, eb: int) -> tuple[int, int]:
    """[first, last + 1) bytes touched by ``rows`` rows of ``width`` elements."""
    return ptr, ptr + ((rows - 1) * stride + width) * eb


def overlaps(a: tuple[int, int], b: tuple[int, int]) -> bool:
    return a[0] < b[1] and b[0] < a[1]


# Buffers placed on a 1 MiB grid, optionally nudged so that ranges can collide.
pointers = st.builds(lambda slot, nudge: 0x10000000 + slot * (1 << 20) + nudge * 2,
                     st.integers(0, 3), st.sampled_from([0, 0, 8, 64, 200]))
small_size = st.integers(0, 6)
width = st.one_of(st.integers(0, 96), st.just(2**31), st.just(2**31 - 1))
stride = st.one_of(st.integers(-8, 160), st.just(0))


@settings(max_examples=400, deadline=None)
@given(x=pointers, r=pointers, w=pointers, y=pointers, ro=pointers, rows=small_size, h=width,
       sx=stride, sr=stride, sy=stride, so=stride, dt=st.sampled_from([0, 1, 2]),
       eps=st.sampled_from([1e-6, 0.0, -1.0, float("nan")]))
def test_rmsnorm_residual_validation_follows_the_contract(x, r, w, y, ro, rows, h, sx, sr, sy, so, dt, eps):
    lib = _native.load()
    status = lib.ako_rmsnorm_residual_fwd(x, r, w, y, ro, rows, h, sx, sr, sy, so, eps, dt, dt, None)
    if rows == 0 or h == 0:
        assert status == 0
        return
    eb = EB[dt]
    reject = (
        h > 2**31 - 1 or not (eps >= 0.0) or min(sx, sr, sy, so) < 0
        or (rows > 1 and (sy < h or so < h))
    )
    if not reject:
        xs, rs, ys, os_ = (byte_range(p, rows, h, s, eb) for p, s in ((x, sx), (r, sr), (y, sy), (ro, so)))
        ws = byte_range(w, 1, h, h, eb)
        reject = any(overlaps(a, b) for a, b in (
            (ys, xs), (ys, rs), (ys, ws), (os_, xs), (os_, rs), (os_, ws), (os_, ys)))
    assert status == (INVALID if reject else NO_DEVICE), (status, _native.last_error())


@settings(max_examples=300, deadline=None)
@given(g=pointers, u=pointers, y=pointers, rows=small_size, n=width, sg=stride, su=stride, sy=stride,
       dt=st.sampled_from([0, 1, 2]))
def test_swiglu_validation_follows_the_contract(g, u, y, rows, n, sg, su, sy, dt):
    lib = _native.load()
    status = lib.ako_swiglu_fwd(g, u, y, rows, n, sg, su, sy, dt, None)
    if rows == 0 or n == 0:
        assert status == 0
        return
    eb = EB[dt]
    reject = n > 2**31 - 1 or min(sg, su, sy) < 0 or (rows > 1 and sy < n)
    if not reject:
        ys = byte_range(y, rows, n, sy, eb)
        reject = overlaps(ys, byte_range(g, rows, n, sg, eb)) or overlaps(ys, byte_range(u, rows, n, su, eb))
    assert status == (INVALID if reject else NO_DEVICE), (status, _native.last_error())
