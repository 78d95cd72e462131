"""Pins the CPU oracle (``oracle.ops``) before any kernel is compared with it.

Each oracle function is checked against something it does not restate:
closed forms evaluated in float64 with the ``math`` module
(``tests/golden/known_answers.json``), golden values the reference repository
records (``tests/golden/reference_golden.json``), invariants the mathematics
fixes (orthogonality, identities, exact zeros), float64 error bounds, and
PyTorch's own rounding for the storage conversions. The last test plants
plausible mistakes in copies of the oracle and requires these checks to catch
every one.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ops
from tests._util import to_np

GOLDEN = Path(__file__).resolve().parent / "golden"
KNOWN = json.loads((GOLDEN / "known_answers.json").read_text())
REF = json.loads((GOLDEN / "reference_golden.json").read_text())
U = {"float32": 2.0**-24, "float16": 2.0**-11, "bfloat16": 2.0**-8}


# -- storage conversions -------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.filterwarnings("ignore:overflow encountered in cast")
def test_round_to_matches_torch_rne(dtype: torch.dtype) -> None:
    g = torch.Generator().manual_seed(0)
    vals = torch.cat([
        torch.randn(100_000, generator=g) * 10,
        torch.randn(1000, generator=g) * 1e-6,
        torch.tensor([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 1e30, -1e30, float("inf"), -float("inf")]),
        # exact ties of the bf16 and fp16 grids
        torch.tensor([1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-11, 1.0 + 3 * 2**-11]),
    ])
    name = "float16" if dtype == torch.float16 else "bfloat16"
    np.testing.assert_array_equal(ops.round_to(vals.numpy(), name), to_np(vals.to(dtype)))
    assert np.isnan(ops.to_f32(ops.round_to(np.array([np.nan], np.float32), name), name)[0])
    widened = ops.to_f32(to_np(vals.to(dtype)), name)
    np.testing.assert_array_equal(widened, vals.to(dtype).float().numpy())


# -- RMSNorm ---------------------------------------------------------------------------


def test_rmsnorm_known_answer() -> None:
    case = KNOWN["rmsnorm_3_4"]
    y = ops.rmsnorm(np.array(case["x"], np.float32), np.array(case["w"], np.float32), case["eps"])
    np.testing.assert_allclose(y, case["y"], rtol=2 * U["float32"], atol=0)


def test_rmsnorm_reproduces_reference_rejection_line() -> None:
    """docs/EXTENDING.md:153-175 of the reference: seed 0, x = randn(4096, 2048),
    w = randn(2048), a mean-absolute-value kernel is rejected with these numbers."""
    gold = REF["extending_rejection"]
    torch.manual_seed(0)
    x = torch.randn(4096, 2048).numpy()
    w = torch.randn(2048).numpy()
    ref = ops.rmsnorm(x, w, 1e-6)
    mean_abs = np.abs(x).sum(-1, keepdims=True, dtype=np.float32) * np.float32(1 / 2048)
    wrong = (x * (np.float32(1) / np.sqrt(mean_abs + np.float32(1e-6)))) * w
    rep = ops.gate(ref, wrong, "float32")
    assert f"{rep['max_error']:.3e}" == gold["max_error"]
    assert f"{rep['budget']:.3e}" == gold["budget"]
    # The count is in fp32 ulps of max|ref| (2**-20 here); reduction order may move it a few.
    assert abs(rep["err_ulps"] - float(gold["ulps"])) <= 4.0


WIDTHS = [3, 5, 7, 100, 257, 1000, 1023, 2049, 4095]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("n", WIDTHS)
def test_rmsnorm_within_fp64_error_bound(n: int, dtype: str) -> None:
    """|oracle - exact| <= (u + (1+u) d32)|y| + eta: the bound the reference proves for
    its own rmsnorm_ref (tests/test_numerical_bounds.py:85-101 of the reference)."""
    rng = np.random.default_rng(n)
    x = ops.round_to(rng.standard_normal((4, n)).astype(np.float32) * 3, dtype)
    w = ops.round_to(1 + 0.1 * rng.standard_normal(n).astype(np.float32), dtype)
    xd = ops.to_f32(x, dtype).astype(np.float64)
    wd = ops.to_f32(w, dtype).astype(np.float64)
    exact = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6) * wd
    u32 = U["float32"]
    gamma = (n + 2) * u32 / (1 - (n + 2) * u32)
    delta32 = (1 - gamma) ** -0.5 * (1 + u32) ** 4 - 1
    u = U[dtype]
    eta = {"float16": 2.0**-24, "bfloat16": 2.0**-133, "float32": 2.0**-149}[dtype]
    bound = (u + (1 + u) * delta32) * np.abs(exact) + eta
    got = ops.to_f32(ops.rmsnorm(x, w, 1e-6, dtype=dtype), dtype).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bound)


def test_rmsnorm_residual_is_storage_add_then_norm() -> None:
    rng = np.random.default_rng(3)
    for dtype in ("float16", "bfloat16", "float32"):
        x = ops.round_to(rng.standard_normal((8, 300)).astype(np.float32), dtype)
        r = ops.round_to(rng.standard_normal((8, 300)).astype(np.float32), dtype)
        w = ops.round_to(rng.standard_normal(300).astype(np.float32), dtype)
        y, s = ops.rmsnorm_residual(x, r, w, dtype=dtype)
        # The sum rounds once to the storage dtype (what x + r does in PyTorch).
        xt, rt = torch.from_numpy(ops.to_f32(x, dtype)), torch.from_numpy(ops.to_f32(r, dtype))
        tdt = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}[dtype]
        np.testing.assert_array_equal(s, to_np(xt.to(tdt) + rt.to(tdt)))
        np.testing.assert_array_equal(y, ops.rmsnorm(s, w, dtype=dtype))
    with pytest.raises(ValueError):
        ops.rmsnorm_residual(np.zeros((2, 8), np.float32), np.zeros((2, 4), np.float32), np.ones(8, np.float32))


# -- RoPE ------------------------------------------------------------------------------


def test_rope_tables_known_values() -> None:
    case = KNOWN["rope_tables_s4_d8"]
    cos, sin = ops.rope_tables(case["seq"], case["head_dim"], base=case["base"])
    # fp32 angle formation: error grows with the angle (|angle| <= 3 here).
    np.testing.assert_allclose(cos, case["cos"], atol=8 * U["float32"] * 3, rtol=0)
    np.testing.assert_allclose(sin, case["sin"], atol=8 * U["float32"] * 3, rtol=0)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    assert cos[1, 0] == pytest.approx(math.cos(1.0), abs=1e-6)
    with pytest.raises(ValueError):
        ops.rope_tables(4, 7)


def test_rope_tables_offset_is_a_shift() -> None:
    full_c, full_s = ops.rope_tables(40, 16)
    off_c, off_s = ops.rope_tables(8, 16, offset=32)
    np.testing.assert_array_equal(off_c, full_c[32:])
    np.testing.assert_array_equal(off_s, full_s[32:])


@pytest.mark.parametrize("style", ["neox", "interleaved"])
def test_rope_rotation_known_answer(style: str) -> None:
    case = KNOWN["rope_rotate_pos3_d8"]
    tables = KNOWN["rope_tables_s4_d8"]
    x = np.zeros((1, 4, 1, 8), np.float32)
    x[0, case["position"], 0] = case["x"]
    cos = np.array(tables["cos"], np.float32)
    sin = np.array(tables["sin"], np.float32)
    out = ops.rope(x, cos, sin, style)
    np.testing.assert_allclose(out[0, case["position"], 0], case[style], atol=1e-6, rtol=0)


@pytest.mark.parametrize("style", ["neox", "interleaved"])
def test_rope_invariants(style: str) -> None:
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 33, 3, 16)).astype(np.float32)
    cos, sin = ops.rope_tables(33, 16)
    out = ops.rope(x, cos, sin, style)
    # Position 0 is the identity rotation, exactly.
    np.testing.assert_array_equal(out[:, 0], x[:, 0])
    # A rotation preserves the norm of every pair.
    half = 8
    if style == "neox":
        pn_in = np.hypot(x[..., :half], x[..., half:])
        pn_out = np.hypot(out[..., :half], out[..., half:])
    else:
        pn_in = np.hypot(x[..., 0::2], x[..., 1::2])
        pn_out = np.hypot(out[..., 0::2], out[..., 1::2])
    np.testing.assert_allclose(pn_out, pn_in, rtol=8 * U["float32"], atol=1e-6)
    # <R_m q, R_n k> depends only on m - n.
    q = np.repeat(rng.standard_normal((1, 1, 1, 16)).astype(np.float32), 33, axis=1)
    k = np.repeat(rng.standard_normal((1, 1, 1, 16)).astype(np.float32), 33, axis=1)
    qr, kr = ops.rope(q, cos, sin, style), ops.rope(k, cos, sin, style)
    dot_a = float((qr[0, 10, 0].astype(np.float64) * kr[0, 6, 0]).sum())
    dot_b = float((qr[0, 25, 0].astype(np.float64) * kr[0, 21, 0]).sum())
    assert dot_a == pytest.approx(dot_b, abs=1e-4)


def test_rope_rejects_bad_input() -> None:
    cos, sin = ops.rope_tables(4, 8)
    with pytest.raises(ValueError):
        ops.rope(np.zeros((2, 4, 8), np.float32), cos, sin)
    with pytest.raises(ValueError):
        ops.rope(np.zeros((1, 4, 1, 8), np.float32), cos, sin, "unknown-style")


def _brute_rotate(vec: np.ndarray, position: int, style: str, base: float = 10000.0) -> np.ndarray:
    """Float64 rotation of one head vector at ``position``, element by element."""
    d = vec.shape[0]
    half = d // 2
    out = np.empty(d, np.float64)
    for i in range(half):
        theta = position * base ** (-2.0 * i / d)
        c, s = math.cos(theta), math.sin(theta)
        ia, ib = (i, i + half) if style == "neox" else (2 * i, 2 * i + 1)
        a, b = float(vec[ia]), float(vec[ib])
        out[ia] = a * c - b * s
        out[ib] = a * s + b * c
    return out


def _check_cache_against_brute(fn, style: str) -> None:
    rng = np.random.default_rng(21)
    batch, seq, q_heads, kv_heads, d, cache_len, pos = 2, 3, 3, 2, 8, 9, 4
    q = rng.standard_normal((batch, seq, q_heads, d)).astype(np.float32)
    k = rng.standard_normal((batch, seq, kv_heads, d)).astype(np.float32)
    v = rng.standard_normal((batch, seq, kv_heads, d)).astype(np.float32)
    k_cache = rng.standard_normal((batch, kv_heads, cache_len, d)).astype(np.float32)
    v_cache = rng.standard_normal((batch, kv_heads, cache_len, d)).astype(np.float32)
    cos, sin = ops.rope_tables(cache_len, d)
    q_out, new_k, new_v = fn(q, k, v, cos, sin, pos, k_cache, v_cache, style)
    for b in range(batch):
        for s in range(seq):
            for h in range(q_heads):
                np.testing.assert_allclose(q_out[b, s, h], _brute_rotate(q[b, s, h], pos + s, style),
                                           atol=2e-6, rtol=0)
            for h in range(kv_heads):
                np.testing.assert_allclose(new_k[b, h, pos + s], _brute_rotate(k[b, s, h], pos + s, style),
                                           atol=2e-6, rtol=0)
                np.testing.assert_array_equal(new_v[b, h, pos + s], v[b, s, h])
    untouched = [t for t in range(cache_len) if not pos <= t < pos + seq]
    np.testing.assert_array_equal(new_k[:, :, untouched], k_cache[:, :, untouched])
    np.testing.assert_array_equal(new_v[:, :, untouched], v_cache[:, :, untouched])


@pytest.mark.parametrize("style", ["neox", "interleaved"])
def test_rope_qk_cache_matches_brute_force(style: str) -> None:
    """Slot placement, table row and rotation of the cache composition, against
    an element-by-element float64 loop over math.cos / math.sin."""
    _check_cache_against_brute(ops.rope_qk_cache, style)


def test_rope_qk_cache_drops_out_of_range_tokens() -> None:
    rng = np.random.default_rng(22)
    q = rng.standard_normal((1, 4, 1, 8)).astype(np.float32)
    k = rng.standard_normal((1, 4, 1, 8)).astype(np.float32)
    kc = np.zeros((1, 1, 6, 8), np.float32)
    cos, sin = ops.rope_tables(6, 8)
    q_out, new_k, new_v = ops.rope_qk_cache(q, k, None, cos, sin, 4, kc, None)
    assert new_v is None
    # slots 4, 5 kept; 6, 7 outside the cache: no slot written, q rows NaN
    assert not np.isnan(q_out[:, :2]).any() and np.any(q_out[:, :2])
    assert np.isnan(q_out[:, 2:]).all()
    assert np.any(new_k[:, :, 4:]) and not np.any(new_k[:, :, :4])


def test_rope_qk_cache_planted_mistakes_are_caught() -> None:
    """Writing at slot s instead of pos + s, or reading table row s, must fail."""

    def wrong_slot(q, k, v, cos, sin, pos, k_cache, v_cache, style):
        q_out, _, _ = ops.rope_qk_cache(q, k, v, cos, sin, pos, k_cache, v_cache, style)
        _, new_k, new_v = ops.rope_qk_cache(q, k, v, cos, sin, 0, k_cache, v_cache, style)
        return q_out, new_k, new_v

    def wrong_row(q, k, v, cos, sin, pos, k_cache, v_cache, style):
        shifted_c = np.roll(cos, pos, axis=0)
        shifted_s = np.roll(sin, pos, axis=0)
        return ops.rope_qk_cache(q, k, v, shifted_c, shifted_s, pos, k_cache, v_cache, style)

    for planted in (wrong_slot, wrong_row):
        with pytest.raises(AssertionError):
            _check_cache_against_brute(planted, "neox")


# -- SwiGLU ----------------------------------------------------------------------------


def test_swiglu_known_answers_and_zero() -> None:
    case = KNOWN["silu"]
    g = np.array(case["g"], np.float32)
    np.testing.assert_allclose(ops.swiglu(g, np.ones_like(g)), case["silu"], rtol=4 * U["float32"], atol=1e-30)
    rng = np.random.default_rng(4)
    assert not np.any(ops.swiglu(rng.standard_normal((3, 16)).astype(np.float32), np.zeros((3, 16), np.float32)))
    with pytest.raises(ValueError):
        ops.swiglu(np.zeros((2, 8), np.float32), np.zeros((2, 16), np.float32))


def test_swiglu_fp32_within_two_ulp_of_float64() -> None:
    """fp32 silu(g) is at most 2 ulp from the float64 value rounded to fp32,
    over [-87, 87] (exp overflows fp32 beyond). Three correctly rounded steps
    (exp, 1 + e, the division) stay within that; numpy's float32 ``exp`` in
    their place, up to 2 ulp off by itself, reaches 3 ulp here."""
    def ordered(a: np.ndarray) -> np.ndarray:
        i = a.view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)

    g = np.linspace(-87.0, 87.0, 1_400_001).astype(np.float32)
    g64 = g.astype(np.float64)
    truth = (g64 / (1.0 + np.exp(-g64))).astype(np.float32)
    got = ops.swiglu(g, np.ones_like(g))
    assert np.abs(ordered(got) - ordered(truth)).max() <= 2
    # Deep in the negative range 1 + e rounds to e: one division of g by the
    # exponential, so any error there is the exponential's own.
    neg = g < -17
    assert np.abs(ordered(got[neg]) - ordered(truth[neg])).max() <= 2


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_swiglu_first_order_bound(dtype: str) -> None:
    """Reference tests/test_numerical_bounds.py:140-151: the half-precision result is
    within 1.05 (kappa + 1) u |y| of the exact one, kappa the condition of silu."""
    rng = np.random.default_rng(5)
    g = rng.standard_normal(4000) * 4
    v = rng.standard_normal(4000)
    g = np.sign(g) * np.maximum(np.abs(g), 1e-3)
    v = np.sign(v) * np.maximum(np.abs(v), 1e-3)
    exact = g / (1 + np.exp(-g)) * v
    got = ops.to_f32(ops.swiglu(ops.round_to(g, dtype), ops.round_to(v, dtype), dtype=dtype), dtype)
    sig = 1 / (1 + np.exp(-g))
    kappa = np.abs(1 + g * (1 - sig))
    # Inputs are rounded (kappa u + u) and the output is rounded once more (u,
    # or half the subnormal spacing once |y| drops below the normal range).
    eta = {"float16": 2.0**-25, "bfloat16": 2.0**-134}[dtype]
    bound = 1.05 * (kappa + 2) * U[dtype] * np.abs(exact) + eta
    assert np.all(np.abs(got - exact) <= bound)


# -- the gate --------------------------------------------------------------------------


def test_ulp_known_answers() -> None:
    for dtype, magnitude, expected in REF["ulp_known_answers"]["cases"]:
        assert ops.ulp(dtype, magnitude) == pytest.approx(expected)
    assert ops.ulp("bfloat16", 0.0) > 0


# -- planted mistakes: every one must be caught ---------------------------------------------


def _known_answer_checks(o) -> list[str]:
    """Run the known-answer / invariant checks against an oracle-like module."""
    failures = []
    case = KNOWN["rmsnorm_3_4"]
    y = o.rmsnorm(np.array(case["x"], np.float32), np.array(case["w"], np.float32), case["eps"])
    if not np.allclose(y, case["y"], rtol=1e-6, atol=0):
        failures.append("rmsnorm")
    t = KNOWN["rope_tables_s4_d8"]
    c, s = o.rope_tables(4, 8)
    if not (np.allclose(c, t["cos"], atol=1e-6) and np.allclose(s, t["sin"], atol=1e-6)):
        failures.append("tables")
    rot = KNOWN["rope_rotate_pos3_d8"]
    x = np.zeros((1, 4, 1, 8), np.float32)
    x[0, 3, 0] = rot["x"]
    for style in ("neox", "interleaved"):
        out = o.rope(x, np.array(t["cos"], np.float32), np.array(t["sin"], np.float32), style)
        if not np.allclose(out[0, 3, 0], rot[style], atol=1e-6):
            failures.append(f"rope_{style}")
    sg = KNOWN["silu"]
    if not np.allclose(o.swiglu(np.array(sg["g"], np.float32), np.ones(len(sg["g"]), np.float32)),
                       sg["silu"], rtol=1e-6, atol=1e-30):
        failures.append("swiglu")
    return failures


def test_checks_pass_on_the_oracle() -> None:
    assert _known_answer_checks(ops) == []


def test_checks_catch_planted_mistakes() -> None:
    import types

    def variant(**overrides):
        mod = types.SimpleNamespace(**{k: getattr(ops, k) for k in ("rmsnorm", "rope_tables", "rope", "swiglu")})
        for k, v in overrides.items():
            setattr(mod, k, v)
        return mod

    def rms_no_mean(x, w, eps=1e-6, **kw):  # sum instead of mean
        xf = x.astype(np.float32)
        return (xf / np.sqrt((xf * xf).sum(-1, keepdims=True) + eps)) * w

    def rope_sign_flip(x, cos, sin, style="neox", **kw):  # rotates the wrong way
        return ops.rope(x, cos, -sin, style, **kw)

    def rope_swapped_styles(x, cos, sin, style="neox", **kw):
        return ops.rope(x, cos, sin, "interleaved" if style == "neox" else "neox", **kw)

    def tables_wrong_exponent(seq, head_dim, **kw):  # i/D instead of 2i/D
        half = head_dim // 2
        inv = 1.0 / np.power(10000.0, np.arange(half) / head_dim)
        ang = np.outer(np.arange(seq), inv).astype(np.float32)
        return np.cos(ang), np.sin(ang)

    def swiglu_sigmoid_only(g, u, **kw):  # drops the gate factor
        return (1 / (1 + np.exp(-g))) * u

    planted = {
        "rmsnorm": variant(rmsnorm=rms_no_mean),
        "rope_sign": variant(rope=rope_sign_flip),
        "rope_styles": variant(rope=rope_swapped_styles),
        "tables": variant(rope_tables=tables_wrong_exponent),
        "swiglu": variant(swiglu=swiglu_sigmoid_only),
    }
    for name, mod in planted.items():
        assert _known_answer_checks(mod), f"planted mistake {name} went unnoticed"
