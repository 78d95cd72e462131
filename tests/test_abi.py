"""The C ABI of libako_hip.so, exercised without a GPU.

The library must load, export every function ``include/ako_hip.h`` declares,
be bound to the HIP runtime PyTorch uses, and reject bad arguments with the
documented status codes before any HIP call is made (all pointers below are
fake addresses that the validation layer never dereferences).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from ako_amd import _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "ako_hip.h"
OK, INVALID, UNSUPPORTED = 0, 1, 2
F32, F16, BF16 = 0, 1, 2
A, B, C, D, E = 0x100000, 0x200000, 0x300000, 0x400000, 0x500000

# Tests that hand the entry points the fake addresses above rely on the
# validation layer refusing the call before any launch. Where a GPU is
# visible a regression there would launch a kernel on those addresses, so
# they run only where no GPU can be launched on (the CPU suite).
fake_addresses = pytest.mark.skipif(
    torch.cuda.is_available(),
    reason="passes fake device addresses: runs only where no GPU is visible")


@pytest.fixture(scope="module")
def lib():
    return _native.load()


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(ako_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_abi() -> None:
    names = declared_functions()
    assert {"ako_rmsnorm_fwd", "ako_rmsnorm_residual_fwd", "ako_rope_fwd", "ako_rope_qk_fwd",
            "ako_rope_qk_cache_fwd", "ako_swiglu_fwd", "ako_last_error", "ako_abi_version"} <= set(names)


def test_library_exports_every_declared_symbol(lib) -> None:
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(_native.SIGNATURES)


def test_versions(lib) -> None:
    assert lib.ako_abi_version() == _native.ABI_VERSION
    version = lib.ako_hip_runtime_version()
    if torch.version.hip:
        assert version == _native._expected_runtime_version()
    assert b"gfx950" in lib.ako_build_info()


def rms(lib, **kw):
    args = dict(x=A, w=B, y=C, rows=4, hidden=64, sx=64, sy=64, eps=1e-6, dt=F16, wdt=F16)
    args.update(kw)
    return lib.ako_rmsnorm_fwd(args["x"], args["w"], args["y"], args["rows"], args["hidden"],
                               args["sx"], args["sy"], args["eps"], args["dt"], args["wdt"], None)


@fake_addresses
def test_rmsnorm_validation(lib) -> None:
    assert rms(lib, rows=0) == OK
    assert rms(lib, hidden=0) == OK
    assert rms(lib, dt=5) == UNSUPPORTED
    assert rms(lib, dt=F16, wdt=BF16) == UNSUPPORTED
    assert rms(lib, rows=-1) == INVALID
    assert rms(lib, x=None) == INVALID
    assert "null pointer" in _native.last_error()
    assert rms(lib, y=A + 64) == INVALID  # y overlaps x
    assert "overlaps" in _native.last_error()
    assert rms(lib, sy=32) == INVALID  # output rows overlap
    assert rms(lib, eps=-1.0) == INVALID
    assert rms(lib, eps=float("nan")) == INVALID
    assert rms(lib, hidden=2**31, sx=2**31, sy=2**31) == INVALID
    assert rms(lib, sx=-64) == INVALID


@fake_addresses
def test_rmsnorm_residual_validation(lib) -> None:
    f = lib.ako_rmsnorm_residual_fwd
    base = [A, B, E, C, D, 4, 64, 64, 64, 64, 64, 1e-6, BF16, F32, None]
    assert f(*base[:5], 0, *base[6:]) == OK
    bad = list(base)
    bad[4] = A  # residual_out aliases x
    assert f(*bad) == INVALID and "residual_out" in _native.last_error()
    bad = list(base)
    bad[1] = None
    assert f(*bad) == INVALID


def rope(lib, **kw):
    a = dict(x=A, cos=B, sin=C, y=D, b=1, s=4, h=2, d=8, xs=(64, 16, 8), ys=(64, 16, 8), st=4,
             dt=F16, tdt=F32, style=0)
    a.update(kw)
    return lib.ako_rope_fwd(a["x"], a["cos"], a["sin"], a["y"], a["b"], a["s"], a["h"], a["d"],
                            *a["xs"], *a["ys"], a["st"], a["dt"], a["tdt"], a["style"], None)


@fake_addresses
def test_rope_validation(lib) -> None:
    assert rope(lib, b=0) == OK
    assert rope(lib, h=0) == OK
    assert rope(lib, d=7) == INVALID and "even" in _native.last_error()
    assert rope(lib, style=3) == UNSUPPORTED
    assert rope(lib, tdt=9) == UNSUPPORTED
    assert rope(lib, cos=None) == INVALID
    assert rope(lib, y=B) == INVALID  # output over the cos table
    assert rope(lib, y=A) == INVALID  # output over the input
    assert rope(lib, ys=(64, 8, 8)) == INVALID  # output tokens overlap
    assert rope(lib, st=2) == INVALID  # table rows shorter than head_dim/2


@fake_addresses
def test_rope_qk_validation(lib) -> None:
    s = (ctypes.c_int64 * 3)(64, 16, 8)
    f = lib.ako_rope_qk_fwd
    assert f(A, B, C, D, E, E + 16, 1, 4, 2, 2, 8, s, s, s, s, 4, F16, F32, 0, None) == INVALID
    assert "two outputs overlap" in _native.last_error()
    assert f(A, B, C, D, E, 0x600000, 0, 4, 2, 2, 8, s, s, s, s, 4, F16, F32, 0, None) == OK
    assert f(A, None, C, D, E, 0x600000, 1, 4, 2, 2, 8, s, s, s, s, 4, F16, F32, 0, None) == INVALID


@fake_addresses
def test_rope_qk_cache_validation(lib) -> None:
    """KV-cache RoPE: argument checks that run before any launch."""
    f = lib.ako_rope_qk_cache_fwd
    tok = (ctypes.c_int64 * 3)(16, 16, 8)          # q/k/v/q_out: (batch, seq, head)
    heads_major = (ctypes.c_int64 * 3)(256, 8, 128)  # cache (batch, slot, head) of [1, 2, 16, 8]
    Q, K, V, COS, SIN, QO, KC, VC, POS = (0x100000 * i for i in range(1, 10))

    def call(*, v=V, vc=VC, pos=POS, kc=KC, cache=heads_major, cache_len=16, rows=16, batch=1):
        return f(Q, K, v, COS, SIN, QO, kc, vc, pos, batch, 1, 2, 2, 8, tok, tok, tok, tok, cache,
                 cache_len, rows, 4, F16, F32, 0, None)

    assert call(batch=0) == OK
    assert call(pos=None) == INVALID and "pos" in _native.last_error()
    assert call(vc=None) == INVALID and "v_cache" in _native.last_error()
    assert call(rows=15) == INVALID and "fewer than cache_len" in _native.last_error()
    assert call(cache_len=0) == INVALID
    assert call(vc=KC + 64) == INVALID and "two outputs overlap" in _native.last_error()
    slots_overlap = (ctypes.c_int64 * 3)(256, 4, 128)
    assert call(cache=slots_overlap) == INVALID and "overlap" in _native.last_error()
    assert call(kc=POS - 16) == INVALID and "pos" in _native.last_error()
    assert call(kc=COS) == INVALID and "table" in _native.last_error()


@fake_addresses
def test_swiglu_validation(lib) -> None:
    f = lib.ako_swiglu_fwd
    assert f(A, B, C, 0, 16, 16, 16, 16, BF16, None) == OK
    assert f(A, B, A, 4, 16, 16, 16, 16, BF16, None) == INVALID
    assert f(A, B, C, 4, 2**31, 2**31, 2**31, 2**31, BF16, None) == INVALID
    assert f(A, B, C, 4, 16, 16, 16, 8, BF16, None) == INVALID
    assert f(A, B, C, 4, 16, 16, 16, 16, 7, None) == UNSUPPORTED
    assert f(None, B, C, 4, 16, 16, 16, 16, BF16, None) == INVALID


@fake_addresses
def test_sizes_that_overflow_the_address_space_are_rejected(lib) -> None:
    """Extents are computed in 128 bits: huge sizes or strides cannot wrap into
    a small span that would pass the overlap checks."""
    big = 2**40
    assert rms(lib, rows=big, sx=2**30, sy=2**30) == INVALID
    assert "overflow" in _native.last_error()
    assert rms(lib, rows=2, sx=2**62, sy=64) == INVALID and "overflow" in _native.last_error()
    assert lib.ako_swiglu_fwd(A, B, C, 2**50, 2**20, 2**20, 2**20, 2**20, BF16, None) == INVALID
    assert "overflow" in _native.last_error()
    huge = (ctypes.c_int64 * 3)(2**61, 16, 8)
    ok = (ctypes.c_int64 * 3)(64, 16, 8)
    assert lib.ako_rope_qk_fwd(A, B, C, D, E, 0x600000, 2, 4, 2, 2, 8, huge, ok, ok, ok, 4, F16, F32, 0,
                               None) == INVALID
    assert "overflow" in _native.last_error()


def test_tuning_keys(lib) -> None:
    assert lib.ako_set_tuning(9, 1, 1) == INVALID
    assert lib.ako_set_tuning(0, 1, -1) == INVALID
    assert lib.ako_set_tuning(0, 5, 3) == INVALID
    assert lib.ako_set_tuning(2, 3, 1) == INVALID  # SwiGLU has two keys: packets per lane, XCD runs
    assert lib.ako_set_tuning(0, 8, 3) == INVALID  # early weights: 0, 1 or 2
    assert lib.ako_set_tuning(0, 9, 3) == INVALID  # pipelined kernel: 0, 1 or 2
    assert lib.ako_set_tuning(0, 10, 33) == INVALID  # pipelined workgroups per CU: at most 32
    assert lib.ako_set_tuning(0, 11, 3) == INVALID  # load groups: 0, 1 or 2
    assert lib.ako_set_tuning(0, 12, 3) == INVALID  # write-through stores: 0, 1 or 2
    assert lib.ako_set_tuning(1, 4, 0) == INVALID  # RoPE has three keys
    for op, key in ((0, 1), (0, 2), (0, 3), (0, 4), (0, 5), (0, 6), (0, 7), (0, 8), (0, 9), (0, 10), (0, 11), (0, 12), (1, 1),
                    (1, 2), (1, 3), (2, 1), (2, 2)):
        assert lib.ako_set_tuning(op, key, 0) == OK


def test_launch_timing_hook_arms_and_disarms(lib) -> None:
    """ako_time_next_launch stores the pair for the calling thread only and
    touches no HIP state: one NULL of the two is refused, disarming reports
    whether a pair was still armed, and a pair armed on another thread is not
    seen here."""
    import threading

    assert lib.ako_time_next_launch(A, None) == INVALID
    assert "both" in _native.last_error()
    assert lib.ako_time_next_launch(None, B) == INVALID
    assert lib.ako_time_next_launch(None, None) == OK  # nothing armed
    assert lib.ako_time_next_launch(A, B) == OK
    assert lib.ako_time_next_launch(C, D) == OK  # replaces the unused pair
    assert lib.ako_time_next_launch(None, None) == 1
    assert lib.ako_time_next_launch(None, None) == OK
    other = threading.Thread(target=lambda: lib.ako_time_next_launch(A, B))
    other.start()
    other.join()
    assert lib.ako_time_next_launch(None, None) == OK


def test_status_codes_become_python_exceptions() -> None:
    with pytest.raises(ValueError, match="ako_x"):
        _native.check(INVALID, "ako_x")
    with pytest.raises(RuntimeError):
        _native.check(3, "ako_x")
    _native.check(OK, "ako_x")


def test_hip_candidates_refuse_cpu_tensors() -> None:
    from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
    from ako_amd.ops.rope_hip import rope_hip, rope_qk_hip
    from ako_amd.ops.rope_ref import build_rope_tables
    from ako_amd.ops.swiglu_hip import swiglu_hip

    x = torch.randn(2, 8, 64)
    cos, sin = build_rope_tables(8, 16)
    q = torch.randn(1, 8, 2, 16)
    for call in (lambda: rmsnorm_hip(x, torch.ones(64)),
                 lambda: rmsnorm_residual_hip(x, x, torch.ones(64)),
                 lambda: rope_hip(q, cos, sin),
                 lambda: rope_qk_hip(q, q, cos, sin),
                 lambda: swiglu_hip(x, x)):
        with pytest.raises(ValueError, match="GPU tensor"):
            call()


def test_missing_library_fails_loudly(monkeypatch, tmp_path) -> None:
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setenv("AKO_HIP_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(_native.HipLibraryError, match="not built"):
        _native.load()
    assert not _native.is_available()


def test_torch_binding_loads_and_checks_like_the_python_wrappers() -> None:
    """The PyTorch binding (``_ako_torch``) is built next to the library, has the
    library's ABI, and rejects what the Python wrappers reject, with the same
    exception type and message (the checks run before any GPU call)."""
    from ako_amd.ops import rmsnorm_hip, rope_hip, swiglu_hip

    fast = _native.torch_binding()
    assert fast is not None and fast.abi_version() == _native.ABI_VERSION
    x, w = torch.zeros(2, 8), torch.ones(8)
    cases = [
        (lambda: fast.rmsnorm(x, w, 1e-6), lambda: rmsnorm_hip.rmsnorm_hip_ctypes(x, w, 1e-6)),
        (lambda: fast.rmsnorm_residual(x, x, w, 1e-6), lambda: rmsnorm_hip.rmsnorm_residual_hip_ctypes(x, x, w)),
        (lambda: fast.swiglu(x, x), lambda: swiglu_hip.swiglu_hip_ctypes(x, x)),
        (lambda: fast.rope(x.view(1, 2, 1, 8), w[:4].view(1, 4).expand(2, 4), w[:4].view(1, 4).expand(2, 4), "neox"),
         lambda: rope_hip.rope_hip_ctypes(x.view(1, 2, 1, 8), w[:4].view(1, 4).expand(2, 4),
                                          w[:4].view(1, 4).expand(2, 4), "neox")),
    ]
    for fast_call, slow_call in cases:
        with pytest.raises(ValueError) as a:
            fast_call()
        with pytest.raises(ValueError) as b:
            slow_call()
        assert str(a.value) == str(b.value) and "GPU tensor" in str(a.value)
