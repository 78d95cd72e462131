"""Unfused PyTorch rotary position embedding, and the rotation tables.

Restates ``ako/ops/rope_ref.py:20-107``. Layout: ``x`` is
``(batch, seq_len, n_heads, head_dim)``, ``cos``/``sin`` are
``(seq_len, head_dim // 2)`` and row ``s`` of the tables rotates position ``s``
of ``x``. Two pairings:

* ``neox`` (GPT-NeoX / HF LLaMA): element ``i`` pairs with ``i + head_dim/2``;
* ``interleaved`` (GPT-J): element ``2i`` pairs with ``2i + 1``.

For a pair ``(a, b)`` rotated by angle ``t``: ``(a cos t - b sin t, a sin t + b cos t)``,
evaluated in fp32 for half-precision inputs, one rounded op at a time.
"""

from __future__ import annotations

import torch

ROPE_STYLES = ("neox", "interleaved")


def build_rope_tables(
    seq_len: int,
    head_dim: int,
    *,
    base: float = 10000.0,
    offset: int = 0,
    device: torch.device | str = "cpu",
    dtype: torch.dtype = torch.float32,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(cos, sin)`` of shape ``(seq_len, head_dim // 2)`` for positions ``offset..``.

    ``inv_freq[i] = 1 / base**(2i / head_dim)`` and the angles
    ``pos * inv_freq`` are formed in fp32 (fp64 when ``dtype`` is fp64), then
    the tables are cast to ``dtype``.
    """
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even, got {head_dim}")
    half = head_dim // 2
    work = torch.float64 if dtype == torch.float64 else torch.float32
    inv_freq = 1.0 / (base ** (torch.arange(0, half, device=device, dtype=work) * 2.0 / head_dim))
    positions = torch.arange(offset, offset + seq_len, device=device, dtype=work)
    angles = torch.outer(positions, inv_freq)
    return angles.cos().to(dtype), angles.sin().to(dtype)


def validate_rope_args(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str) -> None:
    """The reference's argument checks (``rope_ref.py:57-70``), raising ``ValueError``."""
    if style not in ROPE_STYLES:
        raise ValueError(f"Unknown RoPE style '{style}', expected one of {ROPE_STYLES}")
    if x.ndim != 4:
        raise ValueError(
            f"Expected x of shape (batch, seq_len, n_heads, head_dim), got {tuple(x.shape)}"
        )
    head_dim = x.shape[-1]
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even, got {head_dim}")
    if cos.shape != sin.shape:
        raise ValueError(f"cos/sin shape mismatch: {tuple(cos.shape)} vs {tuple(sin.shape)}")
    if cos.shape != (x.shape[1], head_dim // 2):
        raise ValueError(
            f"Expected cos/sin of shape {(x.shape[1], head_dim // 2)}, got {tuple(cos.shape)}"
        )


def rope_ref(
    x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str = "neox"
) -> torch.Tensor:
    validate_rope_args(x, cos, sin, style)
    compute = torch.float32 if x.dtype in (torch.float16, torch.bfloat16) else x.dtype
    xc = x.to(compute)
    c = cos.to(compute)[None, :, None, :]
    s = sin.to(compute)[None, :, None, :]
    if style == "neox":
        half = x.shape[-1] // 2
        a, b = xc[..., :half], xc[..., half:]
        out = torch.cat([a * c - b * s, a * s + b * c], dim=-1)
    else:
        a, b = xc[..., 0::2], xc[..., 1::2]
        out = torch.stack([a * c - b * s, a * s + b * c], dim=-1).flatten(start_dim=-2)
    return out.to(x.dtype)


def rope_qk_ref(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str = "neox"
) -> tuple[torch.Tensor, torch.Tensor]:
    return rope_ref(q, cos, sin, style), rope_ref(k, cos, sin, style)


def rope_qk_cache_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor | None,
    cos: torch.Tensor,
    sin: torch.Tensor,
    pos: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor | None,
    style: str = "neox",
) -> torch.Tensor:
    """RoPE of q and k at positions ``pos[0] + s`` with the keys (and values)
    appended to a heads-major cache, as the unfused composition the
    reference's decoder runs: ``rope(q)``, ``rope(k)`` and the cache append
    (``ako/models/decoder.py:173-177``).

    ``cos``/``sin`` are the full ``(max_positions, head_dim/2)`` tables,
    ``pos`` a one-element int64 tensor, ``k_cache``/``v_cache`` are
    ``(batch, kv_heads, cache_len, head_dim)``. Returns the rotated q; the
    caches are written in place.
    """
    seq = q.shape[1]
    slots = pos.reshape(-1)[:1] + torch.arange(seq, device=pos.device)
    c = cos.index_select(0, slots)
    s = sin.index_select(0, slots)
    q_out = rope_ref(q, c, s, style)
    k_cache.index_copy_(2, slots, rope_ref(k, c, s, style).transpose(1, 2))
    if v is not None:
        v_cache.index_copy_(2, slots, v.transpose(1, 2))
    return q_out
