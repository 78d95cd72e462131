"""LLaMA-style decoder used to turn kernel speedups into end-to-end numbers.

Mirrors ``ako/models/decoder.py:37-335`` of the reference: a stack of
decoder layers on hidden states with two interchangeable backends,

* ``"torch"`` - the unfused eager path (separate residual add, ``rmsnorm_ref``,
  ``rope_ref``, ``F.silu(gate) * up``);
* ``"ako"``   - the same math through the adaptive dispatcher
  (``ako_amd.rmsnorm`` / ``rmsnorm_residual`` / ``rope`` / ``swiglu``), where
  the gfx950 HIP kernels race the PyTorch baselines.

GEMMs and attention stay on PyTorch-ROCm (hipBLASLt, SDPA) in both.

Additions for BASELINE.json configs[4] (the reference stack has no embedding
or head, ``decoder.py:261-266``): ``CausalLM`` adds a token embedding, the
LM head and a greedy decode loop. ``KVCache`` can be preallocated to a
maximum length (``max_len``); appending then writes into the slab instead
of re-concatenating the whole cache on every step as ``torch.cat`` does
(``decoder.py:84-93``); the returned views are the same.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Literal

import torch
import torch.nn.functional as F
from torch import nn

from ako_amd.ops.rmsnorm import rmsnorm, rmsnorm_residual
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref
from ako_amd.ops.rope import rope, rope_qk, rope_qk_cache
from ako_amd.ops.rope_ref import build_rope_tables, rope_ref
from ako_amd.ops.swiglu import swiglu

Backend = Literal["ako", "torch"]
KernelOverride = dict[str, str]


@dataclass
class ModelConfig:
    """Decoder shape (defaults: the reference's TinyLlama-like stack)."""

    hidden_dim: int = 2048
    n_layers: int = 4
    n_heads: int = 32
    n_kv_heads: int = 4
    intermediate_dim: int = 5632
    max_seq_len: int = 2048
    rope_base: float = 10000.0
    rope_style: str = "neox"
    eps: float = 1e-5
    vocab_size: int = 32000
    #: One ``(hidden + 2 * kv_dim) x hidden`` projection for q, k and v instead
    #: of three. The outputs are column slices of one GEMM, which the RoPE
    #: kernels and the caches take as strided views without a copy. At the
    #: configs[4] decode step (hipBLASLt GEMVs, graph-replayed, four layers'
    #: weights) the fused projection takes 92 us per step against 155 us for
    #: three. gate and up stay separate: one 22016-row GEMV ran slower (201 us
    #: against 163 us for the pair).
    fused_qkv: bool = True

    @property
    def head_dim(self) -> int:
        if self.hidden_dim % self.n_heads:
            raise ValueError(f"hidden_dim {self.hidden_dim} is not divisible by n_heads {self.n_heads}")
        return self.hidden_dim // self.n_heads

    def __post_init__(self) -> None:
        if self.n_heads % self.n_kv_heads:
            raise ValueError(f"n_heads {self.n_heads} is not divisible by n_kv_heads {self.n_kv_heads}")
        if self.head_dim % 2:
            raise ValueError(f"head_dim {self.head_dim} must be even for RoPE")


def config5() -> ModelConfig:
    """hidden 4096, 32 heads x 128, FFN 11008, eps 1e-6,
    theta 1e4. Not specified there and chosen here: MHA (32 kv heads, the
    Llama-2-7B geometry that FFN 11008 implies) and a 32000-token vocabulary."""
    return ModelConfig(hidden_dim=4096, n_layers=4, n_heads=32, n_kv_heads=32,
                       intermediate_dim=11008, max_seq_len=1024, rope_base=10000.0,
                       eps=1e-6, vocab_size=32000)


@dataclass
class KVCache:
    """Per-layer key/value cache, laid out ``(batch, seq, kv_heads, head_dim)``."""

    n_layers: int
    max_len: int | None = None
    entries: list[tuple[torch.Tensor, torch.Tensor] | None] = field(default_factory=list)
    lengths: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        if not self.entries:
            self.entries = [None] * self.n_layers
        if not self.lengths:
            self.lengths = [0] * self.n_layers

    @property
    def length(self) -> int:
        return self.lengths[0]

    def slab_tail(self, layer_idx: int, k: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, int]:
        """The next ``k.shape[1]`` free slots of the preallocated slabs, viewed
        heads-major ``(batch, kv_heads, seq, head_dim)`` (the layout
        ``rope_qk_cache`` addresses), and the first of them. Only for a cache
        with ``max_len``."""
        start, add = self.lengths[layer_idx], k.shape[1]
        if start + add > self.max_len:
            raise ValueError(f"KV cache overflow: {start + add} > max_len {self.max_len}")
        slab = self.entries[layer_idx]
        if slab is None:
            shape = (k.shape[0], self.max_len, k.shape[2], k.shape[3])
            slab = (k.new_empty(shape), k.new_empty(shape))
            self.entries[layer_idx] = slab
        end = start + add
        return slab[0][:, start:end].transpose(1, 2), slab[1][:, start:end].transpose(1, 2), start

    def advance(self, layer_idx: int, added: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Count ``added`` tokens written through :meth:`slab_tail`; returns the
        filled part of this layer's cache, ``(batch, seq, heads, dim)``."""
        end = self.lengths[layer_idx] + added
        self.lengths[layer_idx] = end
        slab = self.entries[layer_idx]
        return slab[0][:, :end], slab[1][:, :end]

    def update(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Append ``(k, v)`` and return views of the whole cache of this layer."""
        start, add = self.lengths[layer_idx], k.shape[1]
        if self.max_len is None:
            prev = self.entries[layer_idx]
            if prev is not None:
                k = torch.cat([prev[0], k], dim=1)
                v = torch.cat([prev[1], v], dim=1)
            self.entries[layer_idx] = (k, v)
            self.lengths[layer_idx] = k.shape[1]
            return k, v
        if start + add > self.max_len:
            raise ValueError(f"KV cache overflow: {start + add} > max_len {self.max_len}")
        slab = self.entries[layer_idx]
        if slab is None:
            shape = (k.shape[0], self.max_len, k.shape[2], k.shape[3])
            slab = (k.new_empty(shape), v.new_empty(shape))
            self.entries[layer_idx] = slab
        slab[0][:, start:start + add] = k
        slab[1][:, start:start + add] = v
        self.lengths[layer_idx] = start + add
        return slab[0][:, : start + add], slab[1][:, : start + add]


class StaticKVCache:
    """Fixed-shape key/value cache for HIP-graph-captured decoding.

    Slabs are laid out heads-major, ``(batch, kv_heads, max_len, head_dim)``,
    so attention reads them without a transposed view. The current length
    lives on the device (``pos``), so a decode step has static shapes and can
    be captured once and replayed: keys and values are written at ``pos``
    with ``index_copy_``, attention covers all ``max_len`` slots under an
    additive mask (0 for filled slots, -inf beyond ``pos``), and the RoPE row
    for ``pos`` is gathered from the full table on the device. Multi-token
    calls (prefill) take the host-tracked path with causal attention.
    """

    def __init__(self, n_layers: int, batch: int, kv_heads: int, head_dim: int, max_len: int,
                 *, dtype: torch.dtype, device: torch.device | str) -> None:
        self.n_layers = n_layers
        self.max_len = max_len
        shape = (batch, kv_heads, max_len, head_dim)
        self.k = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(n_layers)]
        self.v = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(n_layers)]
        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        #: Host-side mirror of ``pos``: advanced by every eagerly run step (the
        #: replays of a captured step advance only the device copy, and
        #: ``GraphedGreedy`` sets the mirror after its replays).
        self.host_len = 0
        self.mask = torch.zeros(1, 1, 1, max_len, dtype=dtype, device=device)

    @property
    def length(self) -> int:
        return self.host_len

    def set_length(self, length: int) -> None:
        """Host-side: the first ``length`` slots are filled (after a prefill).
        Sets ``pos`` and the mask: 0 for filled slots, -inf beyond."""
        if length > self.max_len:
            raise ValueError(f"KV cache overflow: {length} > max_len {self.max_len}")
        self.host_len = length
        self.pos.fill_(length)
        self.mask.fill_(float("-inf"))
        self.mask[..., :length] = 0.0

    def begin_step(self) -> None:
        """Open slot ``pos`` in the attention mask for the token being decoded:
        one device-side write per step (capturable). Slots below ``pos`` were
        opened by earlier steps or by ``set_length``. A step past the last slot
        is refused on the host: the device-side index would be out of range."""
        if self.host_len >= self.max_len:
            raise ValueError(f"KV cache overflow: decode step at slot {self.host_len} of {self.max_len}")
        self.mask.index_fill_(-1, self.pos, 0.0)

    def end_step(self, tokens: int) -> None:
        self.pos.add_(tokens)
        self.host_len += tokens

    def rope_rows(self, cos_full: torch.Tensor, sin_full: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return cos_full.index_select(0, self.pos), sin_full.index_select(0, self.pos)

    def update(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor):
        """Store ``(k, v)`` given as ``(batch, seq, heads, dim)``; returns heads-major
        ``(keys, values, mask, causal)`` for attention."""
        n = k.shape[1]
        if n == 1:
            self.k[layer_idx].index_copy_(2, self.pos, k.transpose(1, 2))
            self.v[layer_idx].index_copy_(2, self.pos, v.transpose(1, 2))
            return self.k[layer_idx], self.v[layer_idx], self.mask, False
        start = self.host_len
        if start + n > self.max_len:
            raise ValueError(f"KV cache overflow: {start + n} > max_len {self.max_len}")
        self.k[layer_idx][:, :, start:start + n] = k.transpose(1, 2)
        self.v[layer_idx][:, :, start:start + n] = v.transpose(1, 2)
        end = start + n
        return self.k[layer_idx][:, :, :end], self.v[layer_idx][:, :, :end], None, start == 0


def _norm(backend: Backend, x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor,
          eps: float, override: KernelOverride | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Residual add + RMSNorm, returning ``(normed, residual)``."""
    override = override or {}
    if residual is None:
        if backend == "ako":
            return rmsnorm(x, weight, eps, kernel=override.get("rmsnorm")), x
        return rmsnorm_ref(x, weight, eps), x
    if backend == "ako":
        return rmsnorm_residual(x, residual, weight, eps, kernel=override.get("rmsnorm_residual"))
    residual = x + residual
    return rmsnorm_ref(residual, weight, eps), residual


def _rope(backend: Backend, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, style: str,
          override: KernelOverride | None = None) -> torch.Tensor:
    if backend != "ako":
        return rope_ref(x, cos, sin, style)
    return rope(x, cos, sin, style, kernel=(override or {}).get("rope"))


_ZERO_POSITIONS: dict[torch.device, torch.Tensor] = {}


def _zero_position(device: torch.device) -> torch.Tensor:
    """A one-element int64 zero on ``device``, made once per device."""
    t = _ZERO_POSITIONS.get(device)
    if t is None:
        t = _ZERO_POSITIONS[device] = torch.zeros(1, dtype=torch.long, device=device)
    return t


def _fused_cache_rope(backend: Backend, override: KernelOverride | None) -> bool:
    """Whether a static-cache decode step rotates q/k and appends k/v to the
    cache in one call (``rope_qk_cache``) instead of RoPE plus two copies.
    Forcing a ``rope`` or ``rope_qk`` kernel keeps the unfused path."""
    o = override or {}
    return backend == "ako" and not o.get("rope") and not o.get("rope_qk")


class Attention(nn.Module):
    """Grouped-query attention with RoPE and SDPA."""

    def __init__(self, config: ModelConfig, backend: Backend = "ako",
                 kernel_override: KernelOverride | None = None) -> None:
        super().__init__()
        self.config = config
        self.backend = backend
        self.kernel_override = kernel_override
        self.repeats = config.n_heads // config.n_kv_heads
        kv_dim = config.n_kv_heads * config.head_dim
        self.kv_dim = kv_dim
        if config.fused_qkv:
            self.qkv_proj = nn.Linear(config.hidden_dim, config.hidden_dim + 2 * kv_dim, bias=False)
        else:
            self.q_proj = nn.Linear(config.hidden_dim, config.hidden_dim, bias=False)
            self.k_proj = nn.Linear(config.hidden_dim, kv_dim, bias=False)
            self.v_proj = nn.Linear(config.hidden_dim, kv_dim, bias=False)
        self.o_proj = nn.Linear(config.hidden_dim, config.hidden_dim, bias=False)

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        """State dicts of either layout load into either: three ``q/k/v_proj``
        matrices (the reference's layout, ``ako/models/decoder.py:153-156``)
        are stacked into ``qkv_proj``, and a ``qkv_proj`` is split back."""
        names = [prefix + f"{n}_proj.weight" for n in ("q", "k", "v")]
        fused = prefix + "qkv_proj.weight"
        if self.config.fused_qkv and all(n in state_dict for n in names):
            state_dict[fused] = torch.cat([state_dict.pop(n) for n in names], 0)
        elif not self.config.fused_qkv and fused in state_dict:
            h = self.config.hidden_dim
            q, k, v = state_dict.pop(fused).split([h, self.kv_dim, self.kv_dim], 0)
            for n, t in zip(names, (q, k, v)):
                state_dict[n] = t
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)

    @torch.no_grad()
    def load_qkv(self, q_weight: torch.Tensor, k_weight: torch.Tensor, v_weight: torch.Tensor) -> None:
        """Set the q, k and v projections from three ``(out, hidden)`` matrices
        (e.g. a checkpoint's), whichever layout the module uses."""
        if self.config.fused_qkv:
            self.qkv_proj.weight.copy_(torch.cat([q_weight, k_weight, v_weight], 0))
        else:
            self.q_proj.weight.copy_(q_weight)
            self.k_proj.weight.copy_(k_weight)
            self.v_proj.weight.copy_(v_weight)

    def project_qkv(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``(q, k, v)`` as ``(batch, seq, heads, head_dim)``; strided views of one
        GEMM's output when the projection is fused."""
        batch, seq_len, _ = x.shape
        cfg = self.config
        if cfg.fused_qkv:
            qkv = self.qkv_proj(x)
            h = cfg.hidden_dim
            q = qkv[..., :h].view(batch, seq_len, cfg.n_heads, cfg.head_dim)
            k = qkv[..., h:h + self.kv_dim].view(batch, seq_len, cfg.n_kv_heads, cfg.head_dim)
            v = qkv[..., h + self.kv_dim:].view(batch, seq_len, cfg.n_kv_heads, cfg.head_dim)
            return q, k, v
        q = self.q_proj(x).view(batch, seq_len, cfg.n_heads, cfg.head_dim)
        k = self.k_proj(x).view(batch, seq_len, cfg.n_kv_heads, cfg.head_dim)
        v = self.v_proj(x).view(batch, seq_len, cfg.n_kv_heads, cfg.head_dim)
        return q, k, v

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, layer_idx: int = 0,
                kv_cache: KVCache | None = None) -> torch.Tensor:
        batch, seq_len, _ = x.shape
        cfg = self.config
        q, k, v = self.project_qkv(x)
        if (isinstance(kv_cache, StaticKVCache) and seq_len == 1
                and _fused_cache_rope(self.backend, self.kernel_override)):
            # cos/sin are the full tables here; the position is read on the device.
            q = rope_qk_cache(q, k, v, cos, sin, kv_cache.pos, kv_cache.k[layer_idx],
                              kv_cache.v[layer_idx], cfg.rope_style)
            kh, vh = kv_cache.k[layer_idx], kv_cache.v[layer_idx]
            if self.repeats > 1:
                kh = kh.repeat_interleave(self.repeats, dim=1)
                vh = vh.repeat_interleave(self.repeats, dim=1)
            attn = F.scaled_dot_product_attention(q.transpose(1, 2), kh, vh, attn_mask=kv_cache.mask)
            return self.o_proj(attn.transpose(1, 2).reshape(batch, seq_len, cfg.hidden_dim))
        if (isinstance(kv_cache, KVCache) and kv_cache.max_len is not None
                and _fused_cache_rope(self.backend, self.kernel_override)):
            # Preallocated host-tracked cache: rotate q and write rotated k and v
            # into the slab from the first free slot on, in one call. cos/sin are
            # the rows of positions [start, start + seq), so position 0 of the
            # call is the free slot itself.
            kc, vc, _ = kv_cache.slab_tail(layer_idx, k)
            q = rope_qk_cache(q, k, v, cos, sin, _zero_position(q.device), kc, vc, cfg.rope_style)
            k, v = kv_cache.advance(layer_idx, seq_len)
            return self._attend(q, k, v, batch, seq_len)
        if self.backend == "ako" and not (self.kernel_override or {}).get("rope"):
            # One dispatched op (a single launch on the HIP path) for both tensors.
            q, k = rope_qk(q, k, cos, sin, cfg.rope_style,
                           kernel=(self.kernel_override or {}).get("rope_qk"))
        else:
            q = _rope(self.backend, q, cos, sin, cfg.rope_style, self.kernel_override)
            k = _rope(self.backend, k, cos, sin, cfg.rope_style, self.kernel_override)
        if isinstance(kv_cache, StaticKVCache):
            kh, vh, mask, causal = kv_cache.update(layer_idx, k, v)
            if self.repeats > 1:
                kh = kh.repeat_interleave(self.repeats, dim=1)
                vh = vh.repeat_interleave(self.repeats, dim=1)
            attn = F.scaled_dot_product_attention(q.transpose(1, 2), kh, vh, attn_mask=mask,
                                                  is_causal=causal and mask is None)
            return self.o_proj(attn.transpose(1, 2).reshape(batch, seq_len, cfg.hidden_dim))
        if kv_cache is not None:
            k, v = kv_cache.update(layer_idx, k, v)
        return self._attend(q, k, v, batch, seq_len)

    def _attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, batch: int, seq_len: int) -> torch.Tensor:
        """SDPA over ``(batch, seq, heads, dim)`` q and cached k/v, then the output projection."""
        if self.repeats > 1:
            k = k.repeat_interleave(self.repeats, dim=2)
            v = v.repeat_interleave(self.repeats, dim=2)
        attn = F.scaled_dot_product_attention(
            q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=seq_len > 1
        )
        return self.o_proj(attn.transpose(1, 2).reshape(batch, seq_len, self.config.hidden_dim))


class MLP(nn.Module):
    """SwiGLU feed-forward network."""

    def __init__(self, config: ModelConfig, backend: Backend = "ako",
                 kernel_override: KernelOverride | None = None) -> None:
        super().__init__()
        self.backend = backend
        self.kernel_override = kernel_override
        self.gate_proj = nn.Linear(config.hidden_dim, config.intermediate_dim, bias=False)
        self.up_proj = nn.Linear(config.hidden_dim, config.intermediate_dim, bias=False)
        self.down_proj = nn.Linear(config.intermediate_dim, config.hidden_dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = self.gate_proj(x), self.up_proj(x)
        if self.backend == "ako":
            act = swiglu(gate, up, kernel=(self.kernel_override or {}).get("swiglu"))
        else:
            act = F.silu(gate) * up
        return self.down_proj(act)


class DecoderLayer(nn.Module):
    """norm -> attention -> norm -> MLP, with the residual stream carried along."""

    def __init__(self, config: ModelConfig, layer_idx: int, backend: Backend = "ako",
                 kernel_override: KernelOverride | None = None) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.backend = backend
        self.kernel_override = kernel_override
        self.attention = Attention(config, backend, kernel_override)
        self.mlp = MLP(config, backend, kernel_override)
        self.input_norm_weight = nn.Parameter(torch.ones(config.hidden_dim))
        self.post_attention_norm_weight = nn.Parameter(torch.ones(config.hidden_dim))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None, cos: torch.Tensor,
                sin: torch.Tensor, *, kv_cache: KVCache | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        eps = self.config.eps
        x, residual = _norm(self.backend, x, residual, self.input_norm_weight, eps, self.kernel_override)
        x = self.attention(x, cos, sin, layer_idx=self.layer_idx, kv_cache=kv_cache)
        x, residual = _norm(self.backend, x, residual, self.post_attention_norm_weight, eps,
                            self.kernel_override)
        return self.mlp(x), residual


class DecoderStack(nn.Module):
    """Decoder layers on hidden states (no embedding, no head), final norm."""

    def __init__(self, config: ModelConfig, backend: Backend = "ako",
                 kernel_override: KernelOverride | None = None) -> None:
        super().__init__()
        self.config = config
        self.backend = backend
        self.kernel_override = kernel_override
        self.layers = nn.ModuleList(
            DecoderLayer(config, i, backend, kernel_override) for i in range(config.n_layers)
        )
        self.final_norm_weight = nn.Parameter(torch.ones(config.hidden_dim))
        self._rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None

    def rope_tables(self, seq_len: int, *, offset: int = 0,
                    device: torch.device | str = "cpu") -> tuple[torch.Tensor, torch.Tensor]:
        """fp32 ``(cos, sin)`` for positions ``[offset, offset + seq_len)``, sliced
        from tables built once up to ``max_seq_len``."""
        end = offset + seq_len
        device = torch.device(device)
        cached = self._rope_tables
        if cached is None or cached[0].shape[0] < end or cached[0].device != device:
            self._rope_tables = build_rope_tables(max(end, self.config.max_seq_len), self.config.head_dim,
                                                  base=self.config.rope_base, device=device,
                                                  dtype=torch.float32)
        cos, sin = self._rope_tables
        return cos[offset:end], sin[offset:end]

    def forward(self, x: torch.Tensor, *, kv_cache: KVCache | StaticKVCache | None = None) -> torch.Tensor:
        static_step = isinstance(kv_cache, StaticKVCache) and x.shape[1] == 1
        if static_step:
            full = self.rope_tables(self.config.max_seq_len, device=x.device)
            if _fused_cache_rope(self.backend, self.kernel_override):
                cos, sin = full  # the fused cache RoPE picks row pos itself
            else:
                cos, sin = kv_cache.rope_rows(*full)
            kv_cache.begin_step()
        else:
            offset = kv_cache.length if kv_cache is not None else 0
            cos, sin = self.rope_tables(x.shape[1], offset=offset, device=x.device)
        residual: torch.Tensor | None = None
        for layer in self.layers:
            x, residual = layer(x, residual, cos, sin, kv_cache=kv_cache)
        x, _ = _norm(self.backend, x, residual, self.final_norm_weight, self.config.eps,
                     self.kernel_override)
        if isinstance(kv_cache, StaticKVCache):
            if static_step:
                kv_cache.end_step(1)
            else:
                kv_cache.set_length(kv_cache.host_len + x.shape[1])
        return x

    def new_static_cache(self, max_len: int, *, batch: int = 1) -> StaticKVCache:
        p = next(self.parameters())
        return StaticKVCache(self.config.n_layers, batch, self.config.n_kv_heads, self.config.head_dim,
                             max_len, dtype=p.dtype, device=p.device)

    def new_kv_cache(self, max_len: int | None = None) -> KVCache:
        return KVCache(n_layers=self.config.n_layers, max_len=max_len)


def build_stack(config: ModelConfig, *, backend: Backend = "ako", device: torch.device | str = "cpu",
                dtype: torch.dtype = torch.float32, seed: int = 0,
                kernel_override: KernelOverride | None = None) -> DecoderStack:
    """A stack with reproducible random weights (PyTorch's default init)."""
    torch.manual_seed(seed)
    model = DecoderStack(config, backend=backend, kernel_override=kernel_override)
    return model.to(device=device, dtype=dtype).eval()


class CausalLM(nn.Module):
    """Token embedding -> ``DecoderStack`` -> LM head, with greedy decoding."""

    def __init__(self, config: ModelConfig, backend: Backend = "ako",
                 kernel_override: KernelOverride | None = None) -> None:
        super().__init__()
        self.config = config
        self.embed = nn.Embedding(config.vocab_size, config.hidden_dim)
        self.stack = DecoderStack(config, backend, kernel_override)
        self.lm_head = nn.Linear(config.hidden_dim, config.vocab_size, bias=False)

    def logits_last(self, ids: torch.Tensor, kv_cache: KVCache | None) -> torch.Tensor:
        h = self.stack(self.embed(ids), kv_cache=kv_cache)
        return self.lm_head(h[:, -1])

    @torch.no_grad()
    def generate_greedy(self, prompt: torch.Tensor, steps: int, *,
                        kv_cache: KVCache | None = None) -> torch.Tensor:
        """Prefill ``prompt (batch, seq)`` then ``steps`` argmax tokens; returns them."""
        cache = kv_cache if kv_cache is not None else self.stack.new_kv_cache(prompt.shape[1] + steps)
        nxt = self.logits_last(prompt, cache).argmax(-1, keepdim=True)
        out = [nxt]
        for _ in range(steps - 1):
            nxt = self.logits_last(nxt, cache).argmax(-1, keepdim=True)
            out.append(nxt)
        return torch.cat(out, dim=1)


class GraphedGreedy:
    """Greedy decoding with every decode step replayed from one HIP graph.

    The prompt is prefilled eagerly into a ``StaticKVCache``; one eager decode
    step then runs on a side stream (kernel selection and allocator warmup
    happen there, and its cache slot is rewritten by the first real step),
    and the next step is captured. Each replay reads the token in ``ids``,
    writes the next one back into ``ids`` and into ``history``, and advances
    the device-side position, so decoding needs no host work per token
    beyond the replay call.
    """

    def __init__(self, model: "CausalLM", prompt: torch.Tensor, steps: int) -> None:
        if prompt.shape[0] != 1:
            raise ValueError("graphed decoding is written for batch 1")
        self.model = model
        self.steps = steps
        self.prompt_len = prompt.shape[1]
        max_len = self.prompt_len + steps
        if model.config.max_seq_len < max_len:
            raise ValueError(f"max_seq_len {model.config.max_seq_len} < prompt + steps {max_len}")
        self.cache = model.stack.new_static_cache(max_len)
        self.ids = model.logits_last(prompt, self.cache).argmax(-1, keepdim=True)
        self.history = torch.zeros(steps, dtype=torch.long, device=prompt.device)
        self.history[:1] = self.ids.view(1)
        # After a step, pos has advanced past the token just produced, whose
        # index in history is pos - prompt_len.
        self.base = torch.full((1,), self.prompt_len, dtype=torch.long, device=prompt.device)
        self.slot = torch.zeros(1, dtype=torch.long, device=prompt.device)

        first = self.ids.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._step()
            self.cache.pos.sub_(1)  # undo the warmup step: position and token
            self.cache.host_len -= 1
            self.ids.copy_(first)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        self.cache.host_len -= 1  # capture ran no step on the device
        self._ran = False

    def _step(self) -> None:
        logits = self.model.logits_last(self.ids, self.cache)
        torch.argmax(logits, -1, keepdim=True, out=self.ids)
        torch.sub(self.cache.pos, self.base, out=self.slot)
        self.history.index_copy_(0, self.slot, self.ids.view(1))

    @torch.no_grad()
    def run(self) -> torch.Tensor:
        """Replay the captured step ``steps - 1`` times; once per runner, since
        each replay advances the cache position and the slab holds exactly
        ``prompt + steps`` slots."""
        if self._ran:
            raise RuntimeError("GraphedGreedy.run() decodes once; build a new runner for another pass")
        self._ran = True
        for _ in range(self.steps - 1):
            self.graph.replay()
        self.cache.host_len = self.prompt_len + self.steps - 1
        return self.history.view(1, -1)


def build_lm(config: ModelConfig, *, backend: Backend = "ako", device: torch.device | str = "cpu",
             dtype: torch.dtype = torch.float16, seed: int = 0, init_std: float = 0.02,
             kernel_override: KernelOverride | None = None) -> CausalLM:
    """Random-initialised ``CausalLM``: N(0, init_std) for every Linear and the
    embedding, ones for the norm weights (configs[4]: "random init N(0,0.02)")."""
    torch.manual_seed(seed)
    with torch.device(device):  # initialise in place on the target device
        model = CausalLM(config, backend, kernel_override)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if not name.endswith("norm_weight"):
                p.normal_(0.0, init_std)
    return model.to(dtype=dtype).eval()
