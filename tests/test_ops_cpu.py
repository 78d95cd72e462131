"""The PyTorch references and the public dispatch on the CPU (reference
tests/test_rmsnorm.py, test_rmsnorm_residual.py, test_rope.py, test_swiglu.py,
CPU parts)."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import ako_amd
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref, rmsnorm_residual_ref
from ako_amd.ops.rmsnorm_torch import rmsnorm_torch_native
from ako_amd.ops.rope_ref import build_rope_tables, rope_qk_ref, rope_ref
from ako_amd.ops.swiglu_ref import swiglu_ref
from ako_amd.validation.numerical import assert_close, error_budget, max_abs_error


@pytest.mark.parametrize("shape", [(2, 128, 512), (1, 32, 1024), (4, 64, 256)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rmsnorm_ref_shapes(shape, dtype) -> None:
    x = torch.randn(*shape, dtype=dtype)
    out = rmsnorm_ref(x, torch.ones(shape[-1], dtype=dtype))
    assert out.shape == x.shape and out.dtype == dtype and torch.isfinite(out).all()


def test_rmsnorm_known_value_and_native_baseline() -> None:
    x = torch.tensor([[3.0, 4.0]])
    assert_close(rmsnorm_ref(x, torch.ones(2)), x / torch.sqrt(torch.tensor(12.5)), atol=1e-5, rtol=1e-5)
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        xs, w = torch.randn(2, 32, 128, dtype=dtype), torch.randn(128, dtype=dtype)
        ref = rmsnorm_ref(xs, w)
        assert max_abs_error(ref, rmsnorm_torch_native(xs, w)) < error_budget(ref)


def test_residual_is_the_unfused_composition() -> None:
    x, r, w = torch.randn(2, 16, 64), torch.randn(2, 16, 64), torch.randn(64)
    normed, new_residual = rmsnorm_residual_ref(x, r, w)
    assert_close(new_residual, x + r, atol=0, rtol=0)
    assert_close(normed, rmsnorm_ref(x + r, w), atol=0, rtol=0)
    with pytest.raises(ValueError):
        rmsnorm_residual_ref(torch.randn(2, 8), torch.randn(2, 4), torch.ones(8))


def test_public_dispatch_on_cpu() -> None:
    x, r, w = torch.randn(2, 8, 128), torch.randn(2, 8, 128), torch.ones(128)
    normed, new_residual = ako_amd.rmsnorm_residual(x, r, w)
    ref_normed, ref_residual = rmsnorm_residual_ref(x, r, w)
    assert_close(normed, ref_normed, atol=0, rtol=0)
    assert_close(new_residual, ref_residual, atol=0, rtol=0)
    assert_close(ako_amd.rmsnorm(x, w), rmsnorm_ref(x, w), atol=0, rtol=0)
    with pytest.raises(ValueError, match="Unknown kernel"):
        ako_amd.rmsnorm(x, w, kernel="does_not_exist")
    g, u = torch.randn(2, 8448), torch.randn(2, 8448)
    assert_close(ako_amd.swiglu(g, u), swiglu_ref(g, u), atol=0, rtol=0)
    q = torch.randn(1, 8, 4, 32)
    cos, sin = build_rope_tables(8, 32)
    assert_close(ako_amd.rope(q, cos, sin), rope_ref(q, cos, sin), atol=0, rtol=0)
    qo, ko = ako_amd.rope_qk(q, q, cos, sin, "interleaved")
    assert_close(qo, ko, atol=0, rtol=0)


def test_rope_tables() -> None:
    cos, sin = build_rope_tables(4, 8)
    assert cos.shape == sin.shape == (4, 4)
    assert torch.equal(cos[0], torch.ones(4)) and torch.equal(sin[0], torch.zeros(4))
    assert cos[1, 0].item() == pytest.approx(math.cos(1.0), abs=1e-6)
    with pytest.raises(ValueError):
        build_rope_tables(4, 7)
    full = build_rope_tables(8, 8)
    off = build_rope_tables(4, 8, offset=4)
    assert torch.equal(off[0], full[0][4:]) and torch.equal(off[1], full[1][4:])


@pytest.mark.parametrize("style", ["neox", "interleaved"])
def test_rope_ref_manual_rotation_and_norm(style) -> None:
    x = torch.randn(2, 6, 3, 8)
    cos, sin = build_rope_tables(6, 8)
    out = rope_ref(x, cos, sin, style)
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    if style == "neox":
        assert_close(out[..., :4], x[..., :4] * c - x[..., 4:] * s, atol=1e-6, rtol=1e-6)
    else:
        assert_close(out[..., 1::2], x[..., 0::2] * s + x[..., 1::2] * c, atol=1e-6, rtol=1e-6)
    x64 = torch.randn(1, 12, 2, 16, dtype=torch.float64)
    c64, s64 = build_rope_tables(12, 16, dtype=torch.float64)
    assert_close(rope_ref(x64, c64, s64, style).norm(dim=-1), x64.norm(dim=-1), atol=1e-10, rtol=1e-10)


def test_rope_relative_position_and_errors() -> None:
    q = torch.randn(1, 1, 1, 16, dtype=torch.float64).expand(1, 32, 1, 16).contiguous()
    k = torch.randn(1, 1, 1, 16, dtype=torch.float64).expand(1, 32, 1, 16).contiguous()
    cos, sin = build_rope_tables(32, 16, dtype=torch.float64)
    qr, kr = rope_qk_ref(q, k, cos, sin)
    assert (qr[0, 10] * kr[0, 6]).sum().item() == pytest.approx((qr[0, 25] * kr[0, 21]).sum().item(), abs=1e-8)
    cos4, sin4 = build_rope_tables(4, 8)
    with pytest.raises(ValueError):
        rope_ref(torch.randn(2, 4, 8), cos4, sin4)
    with pytest.raises(ValueError):
        rope_ref(torch.randn(2, 4, 1, 8), cos4[:2], sin4[:2])
    with pytest.raises(ValueError):
        rope_ref(torch.randn(2, 4, 1, 8), cos4, sin4, "unknown-style")


def test_swiglu_ref() -> None:
    g, u = torch.randn(4, 64), torch.randn(4, 64)
    assert_close(swiglu_ref(g, u), F.silu(g) * u, atol=1e-6, rtol=1e-6)
    assert torch.count_nonzero(swiglu_ref(torch.randn(3, 16), torch.zeros(3, 16))) == 0
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        out = swiglu_ref(torch.randn(2, 32, dtype=dtype), torch.randn(2, 32, dtype=dtype))
        assert out.dtype == dtype and torch.isfinite(out).all()
    with pytest.raises(ValueError):
        swiglu_ref(torch.randn(2, 8), torch.randn(2, 16))
