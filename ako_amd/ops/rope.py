"""Public RoPE operations with adaptive kernel selection.

Signatures and dispatch follow ``ako/ops/rope.py:12-58``: ``style`` is part
of the cache key (``extra_key``) and is passed to candidates as a keyword
during selection and positionally afterwards.
"""

from __future__ import annotations

import torch

from ako_amd.dispatcher.selector import get_selector
from ako_amd.ops._registry import hip_disabled, register_all
from ako_amd.ops.rope_ref import build_rope_tables, rope_qk_cache_ref


def rope(
    x: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    style: str = "neox",
    *,
    kernel: str | None = None,
) -> torch.Tensor:
    """Rotate ``x (batch, seq, heads, head_dim)`` by the ``(seq, head_dim/2)`` tables."""
    register_all()
    fn = get_selector().select(
        "rope", x, cos, sin, forced=kernel, extra_key=style, call_kwargs={"style": style}
    )
    return fn(x, cos, sin, style)


def rope_qk(
    q: torch.Tensor,
    k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    style: str = "neox",
    *,
    kernel: str | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE of a query/key pair sharing the tables.

    The reference applies :func:`rope` twice (``ako/ops/rope.py:45-58``);
    here the pair is one dispatched operation, ``rope_qk``, whose HIP
    candidate rotates both tensors in a single launch. The outputs are the
    same as two :func:`rope` calls.
    """
    register_all()
    fn = get_selector().select(
        "rope_qk", q, k, cos, sin, forced=kernel, extra_key=style, call_kwargs={"style": style}
    )
    return fn(q, k, cos, sin, style)


def rope_qk_cache(
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
    """RoPE of q and k at positions ``pos[0] + s``, with the rotated keys and
    the values written into the heads-major caches; returns the rotated q.

    This fuses what the reference's decoder does per layer and step --
    ``rope(q)``, ``rope(k)``, then the cache append
    (``ako/models/decoder.py:173-177``) -- into one launch on a GPU. It is
    not a selector operation: the reference's candidate contract is that
    candidates never write their inputs, and this one writes the caches.
    On a GPU it calls the HIP kernel (and raises if the library cannot be
    loaded, unless ``AKO_HIP_DISABLE=1``); on the CPU it runs the unfused
    composition ``rope_qk_cache_ref``.
    """
    if q.is_cuda and not hip_disabled():
        from ako_amd.ops.rope_hip import rope_qk_cache_hip

        return rope_qk_cache_hip(q, k, v, cos, sin, pos, k_cache, v_cache, style)
    return rope_qk_cache_ref(q, k, v, cos, sin, pos, k_cache, v_cache, style)


__all__ = ["build_rope_tables", "rope", "rope_qk", "rope_qk_cache"]
