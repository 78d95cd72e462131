"""The decoder harness on the CPU (reference tests/test_model.py:21-79)."""

from __future__ import annotations

import pytest
import torch

from ako_amd.models.decoder import KVCache, ModelConfig, build_lm, build_stack, config5
from ako_amd.validation.numerical import assert_close

SMALL = ModelConfig(hidden_dim=64, n_layers=2, n_heads=4, n_kv_heads=2, intermediate_dim=128, max_seq_len=64)


def test_config_validation_and_config5() -> None:
    with pytest.raises(ValueError):
        ModelConfig(hidden_dim=64, n_heads=6, n_kv_heads=3)
    with pytest.raises(ValueError):
        ModelConfig(hidden_dim=64, n_heads=4, n_kv_heads=3)
    c = config5()
    assert (c.hidden_dim, c.n_heads, c.head_dim, c.intermediate_dim, c.eps, c.n_layers) == (4096, 32, 128, 11008, 1e-6, 4)


def test_backends_agree_and_shapes() -> None:
    x = torch.randn(2, 8, SMALL.hidden_dim)
    ako_out = build_stack(SMALL, backend="ako", seed=7)(x)
    torch_out = build_stack(SMALL, backend="torch", seed=7)(x)
    assert ako_out.shape == (2, 8, SMALL.hidden_dim) and torch.isfinite(ako_out).all()
    assert_close(ako_out, torch_out, atol=1e-5, rtol=1e-5)


def test_attention_is_causal() -> None:
    model = build_stack(SMALL, backend="ako", seed=3)
    x = torch.randn(1, 8, SMALL.hidden_dim)
    changed = x.clone()
    changed[:, 5:] += 1.0
    base, other = model(x), model(changed)
    assert_close(base[:, :5], other[:, :5], atol=1e-5, rtol=1e-5)
    assert not torch.allclose(base[:, 5:], other[:, 5:])


@pytest.mark.parametrize("max_len", [None, 16])
def test_kv_cache_decode_matches_prefill(max_len) -> None:
    model = build_stack(SMALL, backend="ako", seed=11)
    x = torch.randn(1, 6, SMALL.hidden_dim)
    prefill = model(x)
    cache = model.new_kv_cache(max_len)
    decoded = torch.cat([model(x[:, i:i + 1], kv_cache=cache) for i in range(6)], dim=1)
    assert cache.length == 6
    assert_close(decoded, prefill, atol=1e-4, rtol=1e-4)


def test_kv_cache_growth_and_overflow() -> None:
    cache = KVCache(n_layers=2)
    k = torch.randn(1, 1, 2, 8)
    cache.update(0, k, k)
    cache.update(0, k, k)
    assert cache.length == 2 and cache.entries[1] is None
    fixed = KVCache(n_layers=1, max_len=2)
    fixed.update(0, k, k)
    kk, _ = fixed.update(0, k, k)
    assert kk.shape[1] == 2
    with pytest.raises(ValueError, match="overflow"):
        fixed.update(0, k, k)


def test_greedy_generation_backends_agree() -> None:
    cfg = ModelConfig(hidden_dim=64, n_layers=2, n_heads=4, n_kv_heads=4, intermediate_dim=96,
                      max_seq_len=32, vocab_size=50, eps=1e-6)
    prompt = torch.randint(0, 50, (1, 7), generator=torch.Generator().manual_seed(0))
    a = build_lm(cfg, backend="ako", dtype=torch.float32, seed=5).generate_greedy(prompt, 6)
    b = build_lm(cfg, backend="torch", dtype=torch.float32, seed=5).generate_greedy(prompt, 6)
    assert a.shape == (1, 6) and torch.equal(a, b)


def test_static_cache_decode_matches_cat_cache() -> None:
    cfg = ModelConfig(hidden_dim=64, n_layers=2, n_heads=4, n_kv_heads=2, intermediate_dim=96,
                      max_seq_len=32, vocab_size=50, eps=1e-6)
    model = build_lm(cfg, backend="ako", dtype=torch.float32, seed=5)
    prompt = torch.randint(0, 50, (1, 7), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        cat_cache = model.stack.new_kv_cache()
        static = model.stack.new_static_cache(16)
        h_cat = model.logits_last(prompt, cat_cache)
        h_static = model.logits_last(prompt, static)
        assert_close(h_static, h_cat, atol=1e-5, rtol=1e-5)
        ids = h_cat.argmax(-1, keepdim=True)
        for _ in range(5):
            a = model.logits_last(ids, cat_cache)
            b = model.logits_last(ids, static)
            assert_close(b, a, atol=1e-5, rtol=1e-5)
            ids = a.argmax(-1, keepdim=True)
    # The host mirror follows the decode steps, so a later multi-token call
    # starts at the true length.
    assert int(static.pos) == 12 and static.length == 12
    with pytest.raises(ValueError, match="overflow"):
        static.update(0, torch.zeros(1, 20, 2, 16), torch.zeros(1, 20, 2, 16))


def test_static_cache_refuses_steps_past_its_slab() -> None:
    """A decode step past the last slot raises on the host before any
    device-side index (the mask slot, the cache slot) could go out of range."""
    cfg = ModelConfig(hidden_dim=64, n_layers=1, n_heads=4, n_kv_heads=4, intermediate_dim=96,
                      max_seq_len=16, vocab_size=50, eps=1e-6)
    model = build_lm(cfg, backend="ako", dtype=torch.float32, seed=6)
    prompt = torch.randint(0, 50, (1, 5), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        static = model.stack.new_static_cache(7)
        ids = model.logits_last(prompt, static).argmax(-1, keepdim=True)
        for _ in range(2):  # slots 5 and 6
            ids = model.logits_last(ids, static).argmax(-1, keepdim=True)
        assert static.length == 7 and int(static.pos) == 7
        with pytest.raises(ValueError, match="overflow"):
            model.logits_last(ids, static)
        assert int(static.pos) == 7  # nothing ran
        with pytest.raises(ValueError, match="overflow"):
            model.stack.new_static_cache(4).set_length(5)


def _hf_pair(n_kv_heads: int, fused_qkv: bool = True):
    """A small Hugging Face LlamaModel (random weights, built offline from a
    config) and this package's stack carrying the same weights."""
    transformers = pytest.importorskip("transformers")
    from ako_amd.models.decoder import DecoderStack

    hf_cfg = transformers.LlamaConfig(hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                                      num_key_value_heads=n_kv_heads, intermediate_size=96, vocab_size=50,
                                      max_position_embeddings=64, rms_norm_eps=1e-6, rope_theta=10000.0)
    hf_cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    hf = transformers.LlamaModel(hf_cfg).eval().to(torch.float32)
    with torch.no_grad():
        for p in hf.parameters():
            p.normal_(0.0, 0.05)
    cfg = ModelConfig(hidden_dim=64, n_layers=2, n_heads=4, n_kv_heads=n_kv_heads, intermediate_dim=96,
                      max_seq_len=64, vocab_size=50, eps=1e-6, rope_base=10000.0, fused_qkv=fused_qkv)
    stacks = {}
    for backend in ("torch", "ako"):
        stack = DecoderStack(cfg, backend).eval()
        with torch.no_grad():
            for ours, theirs in zip(stack.layers, hf.layers):
                att = theirs.self_attn
                ours.attention.load_qkv(att.q_proj.weight, att.k_proj.weight, att.v_proj.weight)
                ours.attention.o_proj.weight.copy_(att.o_proj.weight)
                for name in ("gate_proj", "up_proj", "down_proj"):
                    getattr(ours.mlp, name).weight.copy_(getattr(theirs.mlp, name).weight)
                ours.input_norm_weight.copy_(theirs.input_layernorm.weight)
                ours.post_attention_norm_weight.copy_(theirs.post_attention_layernorm.weight)
            stack.final_norm_weight.copy_(hf.norm.weight)
        stacks[backend] = stack
    return hf, stacks


@pytest.mark.parametrize("fused_qkv", [True, False])
@pytest.mark.parametrize("n_kv_heads", [4, 2])
def test_stack_matches_hugging_face_llama(n_kv_heads: int, fused_qkv: bool) -> None:
    """An independent implementation of the same architecture (the reference's
    tests/test_hf_loader.py compares against it too): hidden states of a
    prompt, and token-by-token decoding through the KV caches, within 1e-5,
    with the q/k/v projections fused into one GEMM or kept as three."""
    hf, stacks = _hf_pair(n_kv_heads, fused_qkv)
    ids = torch.randint(0, 50, (1, 12), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        want = hf(input_ids=ids).last_hidden_state
        emb = hf.embed_tokens(ids)
        for backend, stack in stacks.items():
            assert_close(stack(emb), want, atol=1e-5, rtol=1e-5)
            for cache in (stack.new_kv_cache(), stack.new_kv_cache(16), stack.new_static_cache(16)):
                got = [stack(emb[:, :9], kv_cache=cache)[:, -1]]
                for t in range(9, 12):
                    got.append(stack(emb[:, t:t + 1], kv_cache=cache)[:, -1])
                assert_close(torch.stack(got, 1), want[:, 8:12], atol=1e-5, rtol=1e-5)


def test_state_dicts_load_across_projection_layouts() -> None:
    """A state dict with three q/k/v matrices (the reference's layout) loads
    into the fused model and the other way round; outputs are unchanged."""
    import dataclasses

    separate = build_stack(dataclasses.replace(SMALL, fused_qkv=False), backend="torch", seed=5).eval()
    fused = build_stack(dataclasses.replace(SMALL, fused_qkv=True), backend="torch", seed=9).eval()
    fused.load_state_dict(separate.state_dict())
    x = torch.randn(2, 7, SMALL.hidden_dim)
    with torch.no_grad():
        want = separate(x)
        assert_close(fused(x), want, atol=1e-6, rtol=1e-6)
        back = build_stack(dataclasses.replace(SMALL, fused_qkv=False), backend="torch", seed=11).eval()
        back.load_state_dict(fused.state_dict())
        assert_close(back(x), want, atol=1e-6, rtol=1e-6)
    assert "layers.0.attention.qkv_proj.weight" in fused.state_dict()
    assert "layers.0.attention.q_proj.weight" in back.state_dict()
