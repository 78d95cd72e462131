"""Public RoPE operations with adaptive kernel selection.

Signatures and dispatch follow ``ako/ops/rope.py:12-58``: ``style`` is part
of the cache key (``extra_key``) and is passed to candidates as a keyword
during selection and positionally afterwards.
"""

from __future__ import annotations

import torch

from ako_amd.dispatcher.selector import get_selector
from ako_amd.ops._registry import register_all
from ako_amd.ops.rope_ref import build_rope_tables


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


__all__ = ["build_rope_tables", "rope", "rope_qk"]
