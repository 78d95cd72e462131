"""CPU oracle: numpy restatement of the reference's unfused operations.

TEST INFRASTRUCTURE ONLY. Nothing in the ``ako_amd`` package imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the checker (or the timed CPU
baseline), never as a product code path.

Every function restates one function of Farx1/AKO and follows its order of
fp32 operations, each rounded separately as numpy evaluates them (no fused
multiply-add):

===================  ==========================================  =========
oracle function      reference                                   pinned by
===================  ==========================================  =========
``rmsnorm``          ``ako/ops/rmsnorm_ref.py:8-23``             known answer [[3,4]]; fp64 error bound;
                                                                 golden rejection line of
                                                                 ``docs/EXTENDING.md:153-175``; F.rms_norm
``rmsnorm_residual`` ``ako/ops/rmsnorm_ref.py:26-50``            composition identity; storage-dtype add
``rope_tables``      ``ako/ops/rope_ref.py:20-54``               cos[0]=1, sin[0]=0, cos[1,0]=cos(1);
                                                                 offset shift; fp64 angle bound
``rope``             ``ako/ops/rope_ref.py:73-107``              manual rotation; pair-norm preservation;
                                                                 position-0 identity; relative-position
                                                                 dot product
``rope_qk_cache``    ``ako/models/decoder.py:173-177`` (rope of  element-by-element float64 brute force of
                     q and k, then the cache append of           slot placement, table row and rotation;
                     ``:84-93``), heads-major cache              out-of-range slots dropped; planted
                                                                 wrong-slot / wrong-row mistakes caught
``swiglu``           ``ako/ops/swiglu_ref.py:16-32``             zero-up -> 0; silu closed form in fp64;
                                                                 first-order error bound; fp32 silu
                                                                 within 2 ulp of float64 over [-87, 87]
===================  ==========================================  =========

Storage formats: fp32 arrays are ``float32``, fp16 arrays ``float16``, and
bf16 arrays are ``uint16`` bit patterns (numpy has no bfloat16); ``to_f32``
and ``round_to`` convert with round-to-nearest-even, as PyTorch does.
"""

from __future__ import annotations

import numpy as np

DTYPES = ("float32", "float16", "bfloat16")


# -- storage conversions ---------------------------------------------------------


def to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    """Widen a stored array to float32 (exact for all three formats)."""
    if dtype == "bfloat16":
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    return np.asarray(a).astype(np.float32)


def round_to(a: np.ndarray, dtype: str) -> np.ndarray:
    """Narrow float32 values to the storage format, round-to-nearest-even."""
    a = np.asarray(a, dtype=np.float32)
    if dtype == "float32":
        return a.copy()
    if dtype == "float16":
        with np.errstate(over="ignore"):  # beyond 65504 rounds to inf, as IEEE narrowing does
            return a.astype(np.float16)
    if dtype == "bfloat16":
        bits = a.view(np.uint32).astype(np.uint64)
        lsb = (bits >> 16) & 1
        rounded = ((bits + 0x7FFF + lsb) >> 16).astype(np.uint16)
        return np.where(np.isnan(a), np.uint16(0x7FC0), rounded)
    raise ValueError(f"unknown dtype {dtype}")


# -- RMSNorm --------------------------------------------------------------------------


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, *, dtype: str = "float32",
            w_dtype: str | None = None) -> np.ndarray:
    """``rmsnorm_ref`` (rmsnorm_ref.py:19-23): widen, mean of squares over the last
    axis, ``(x * rsqrt(var + eps)) * w``, narrow to x's dtype.

    The mean is ``sum * fp32(1/H)``, the form PyTorch's mean reduction uses.
    ``rsqrt`` is evaluated as ``1 / sqrt`` in fp32 (both correctly rounded).
    """
    xf = to_f32(x, dtype)
    wf = to_f32(w, w_dtype or dtype)
    hidden = xf.shape[-1]
    if hidden == 0 or xf.size == 0:
        return round_to(xf, dtype)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):  # inf/NaN rows follow IEEE, as on the GPU
        sq = xf * xf
        var = sq.sum(axis=-1, keepdims=True, dtype=np.float32) * np.float32(1.0 / hidden)
        rstd = np.float32(1.0) / np.sqrt(var + np.float32(eps))
        return round_to((xf * rstd) * wf, dtype)


def rmsnorm_residual(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float = 1e-6, *,
                     dtype: str = "float32", w_dtype: str | None = None
                     ) -> tuple[np.ndarray, np.ndarray]:
    """``rmsnorm_residual_ref`` (rmsnorm_ref.py:47-50): the sum ``x + r`` is taken
    in the storage dtype (fp32 add, rounded), then normalised."""
    if np.shape(x) != np.shape(r):
        raise ValueError(f"Shape mismatch: x {np.shape(x)} vs residual {np.shape(r)}")
    with np.errstate(over="ignore", invalid="ignore"):  # inf + -inf is NaN, as on the GPU
        s = round_to(to_f32(x, dtype) + to_f32(r, dtype), dtype)
    return rmsnorm(s, w, eps, dtype=dtype, w_dtype=w_dtype), s


# -- RoPE ---------------------------------------------------------------------------


def rope_tables(seq_len: int, head_dim: int, *, base: float = 10000.0, offset: int = 0,
                dtype: str = "float32") -> tuple[np.ndarray, np.ndarray]:
    """``build_rope_tables`` (rope_ref.py:42-54) with fp32 angle formation:
    ``inv_freq = 1 / base ** (arange(half) * 2 / head_dim)``,
    angles = outer(positions, inv_freq), then cos/sin narrowed to ``dtype``.

    Every step is an fp32 operation rounded once. ``pow``, ``cos`` and ``sin``
    are the correctly rounded fp32 functions (float64 evaluation, one
    rounding), which the reference's 1-ulp fp32 functions approximate;
    numpy's float32 versions would tie the result to the host CPU's SIMD
    code path."""
    if head_dim % 2:
        raise ValueError(f"head_dim must be even, got {head_dim}")
    half = head_dim // 2
    exponent = (np.arange(half, dtype=np.float32) * np.float32(2.0)) / np.float32(head_dim)
    powered = np.power(np.float64(np.float32(base)), exponent.astype(np.float64)).astype(np.float32)
    inv_freq = np.float32(1.0) / powered
    positions = np.arange(offset, offset + seq_len, dtype=np.float32)
    angles = np.outer(positions, inv_freq).astype(np.float32)
    a64 = angles.astype(np.float64)
    return (round_to(np.cos(a64).astype(np.float32), dtype),
            round_to(np.sin(a64).astype(np.float32), dtype))


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, style: str = "neox", *,
         dtype: str = "float32", table_dtype: str = "float32") -> np.ndarray:
    """``rope_ref`` (rope_ref.py:92-107) on ``x (batch, seq, heads, head_dim)``.

    Pairs are ``(i, i + D/2)`` for ``neox`` and ``(2i, 2i+1)`` for
    ``interleaved``; each pair ``(a, b)`` becomes ``(a*c - b*s, a*s + b*c)``.
    """
    if style not in ("neox", "interleaved"):
        raise ValueError(f"Unknown RoPE style '{style}'")
    xf = to_f32(x, dtype)
    if xf.ndim != 4 or xf.shape[-1] % 2:
        raise ValueError(f"Expected (batch, seq, heads, even head_dim), got {xf.shape}")
    c = to_f32(cos, table_dtype)[None, :, None, :]
    s = to_f32(sin, table_dtype)[None, :, None, :]
    half = xf.shape[-1] // 2
    with np.errstate(over="ignore", invalid="ignore"):  # IEEE inf/NaN, as on the GPU
        if style == "neox":
            a, b = xf[..., :half], xf[..., half:]
            out = np.concatenate([a * c - b * s, a * s + b * c], axis=-1)
        else:
            a, b = xf[..., 0::2], xf[..., 1::2]
            out = np.stack([a * c - b * s, a * s + b * c], axis=-1).reshape(xf.shape)
        return round_to(out, dtype)


def rope_qk_cache(q: np.ndarray, k: np.ndarray, v: np.ndarray | None, cos: np.ndarray,
                  sin: np.ndarray, pos: int, k_cache: np.ndarray, v_cache: np.ndarray | None,
                  style: str = "neox", *, dtype: str = "float32",
                  table_dtype: str = "float32") -> tuple[np.ndarray, np.ndarray, np.ndarray | None]:
    """The reference decoder's per-layer ``rope(q)``, ``rope(k)`` and cache
    append (decoder.py:173-177, KVCache.update at :84-93), with the cache laid
    out heads-major ``(batch, kv_heads, cache_len, head_dim)`` and the new
    tokens at slots ``pos .. pos + seq - 1``; the tables are the full
    ``(positions, head_dim/2)`` ones, read at the same rows.

    Returns ``(q_rotated, new_k_cache, new_v_cache)``; the inputs are not
    modified. Tokens whose slot falls outside the cache write no slot, and
    their q rows are NaN: the library's contract where the reference's
    ``index_select`` would raise (a position in device memory cannot raise).
    """
    seq = q.shape[1]
    cache_len = k_cache.shape[2]
    keep = [s for s in range(seq) if 0 <= pos + s < cache_len]
    q_out = round_to(np.full(q.shape, np.nan, np.float32), dtype)
    new_k = k_cache.copy()
    new_v = None if v_cache is None else v_cache.copy()
    if not keep:
        return q_out, new_k, new_v
    rows = np.array([pos + s for s in keep])
    c, sn = cos[rows], sin[rows]
    q_out[:, keep] = rope(q[:, keep], c, sn, style, dtype=dtype, table_dtype=table_dtype)
    k_rot = rope(k[:, keep], c, sn, style, dtype=dtype, table_dtype=table_dtype)
    new_k[:, :, rows] = k_rot.transpose(0, 2, 1, 3)
    if v is not None:
        new_v[:, :, rows] = v[:, keep].transpose(0, 2, 1, 3)
    return q_out, new_k, new_v


# -- SwiGLU -------------------------------------------------------------------------


def swiglu(g: np.ndarray, u: np.ndarray, *, dtype: str = "float32") -> np.ndarray:
    """``swiglu_ref`` (swiglu_ref.py:29-32): ``silu(g) * u`` in fp32 with
    ``silu(g) = g / (1 + exp(-g))``, narrowed to the storage dtype.

    ``exp`` is the correctly rounded fp32 exponential: evaluated in float64
    and rounded once to fp32 (overflowing to inf past the fp32 range). The
    reference's ``F.silu`` calls a 1-ulp fp32 ``exp`` on either device, so the
    correctly rounded value is the one both sides approximate. numpy's own
    float32 ``exp`` is not used: it is up to 2 ulp from the correctly rounded
    value and depends on the host CPU's SIMD code path."""
    if np.shape(g) != np.shape(u):
        raise ValueError(f"Shape mismatch: gate {np.shape(g)} vs up {np.shape(u)}")
    gf = to_f32(g, dtype)
    uf = to_f32(u, dtype)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-gf.astype(np.float64)).astype(np.float32)
        silu = gf / (np.float32(1.0) + e)
        return round_to(silu * uf, dtype)


# -- the gate, for reports ----------------------------------------------------------------

RTOL = {"float64": 1e-7, "float32": 1.3e-6, "float16": 1e-3, "bfloat16": 1.6e-2}
EPS = {"float32": 2.0 ** -23, "float16": 2.0 ** -10, "bfloat16": 2.0 ** -7}
TINY = {"float32": 2.0 ** -126, "float16": 2.0 ** -14, "bfloat16": 2.0 ** -126}


def ulp(dtype: str, magnitude: float) -> float:
    """Spacing of ``dtype`` values in the binade of ``magnitude``
    (``ako/validation/numerical.py:77-88``)."""
    m = abs(float(magnitude))
    if m < TINY[dtype]:
        return TINY[dtype]
    return float(np.ldexp(EPS[dtype], int(np.frexp(m)[1]) - 1))


def gate(ref: np.ndarray, cand: np.ndarray, dtype: str) -> dict[str, float | bool]:
    """``atol + rtol(dtype) * max|ref|`` and the error in ulps of ``max|ref|``
    (``ako/validation/numerical.py:91-122``); arrays in storage format."""
    rf = to_f32(ref, dtype).astype(np.float64)
    cf = to_f32(cand, dtype).astype(np.float64)
    if rf.size == 0:
        return {"max_error": 0.0, "budget": 1e-5, "err_ulps": 0.0, "passed": True, "max_abs_ref": 0.0}
    diff = np.abs(rf - cf)
    # NaN in either output counts as a disagreement unless both are NaN.
    both_nan = np.isnan(rf) & np.isnan(cf)
    diff = np.where(both_nan, 0.0, diff)
    err = float(np.nan_to_num(diff, nan=np.inf).max())
    mag = float(np.abs(np.where(np.isnan(rf), 0.0, rf)).max())
    budget = 1e-5 + RTOL[dtype] * mag
    return {"max_error": err, "budget": budget, "err_ulps": err / ulp(dtype, mag),
            "passed": err <= budget, "max_abs_ref": mag}
