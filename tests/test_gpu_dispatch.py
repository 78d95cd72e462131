"""GPU: dispatch through the public API, HIP-graph capture, decoder backends."""

from __future__ import annotations

import pytest
import torch

import ako_amd
from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.registry import KernelRegistry
from ako_amd.dispatcher.selector import KernelSelector
from ako_amd.ops._registry import register_all
from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
from ako_amd.ops.rope_hip import rope_hip, rope_qk_cache_hip, rope_qk_hip
from ako_amd.ops.rope_ref import build_rope_tables, rope_ref
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref
from ako_amd.ops.swiglu_hip import swiglu_hip
from ako_amd.validation.numerical import error_budget, max_abs_error, max_abs_error_any

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]
DEV = "cuda"


def _rand(*shape, dtype=torch.bfloat16, seed=0, scale=1.0, shift=0.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV) * scale + shift).to(dtype)


def test_selector_picks_hip_and_records_it(tmp_path) -> None:
    sel = KernelSelector(registry=register_all(KernelRegistry()), cache=KernelCache(path=tmp_path / "c.json"))
    x = _rand(2048, 4096, dtype=torch.float16)
    w = _rand(4096, dtype=torch.float16, seed=1, scale=0.1, shift=1.0)
    result = sel.select_entry("rmsnorm", x, w)
    assert result.source == "benchmark"
    assert any(r["kernel"] == "rmsnorm_hip" and r["passed"] for r in result.ulp_reports)
    assert result.entry.kernel_name == "rmsnorm_hip", result.to_dict()
    again = sel.select_entry("rmsnorm", x, w)
    assert again.source == "cache" and again.entry.kernel_name == "rmsnorm_hip"


def test_cache_key_names_the_part() -> None:
    """The selection cache key carries the ISA and CU count that HIP reports,
    and a driver version (never null on a ROCm box)."""
    from ako_amd.dispatcher.hardware import clear_device_cache, get_device_info

    clear_device_cache()
    info = get_device_info("cuda:0")
    print(f"device_name={info.device_name!r} cache_key={info.cache_key!r} driver={info.driver_version!r}")
    assert "gfx950" in info.cache_key and f"{info.sm_count}CU" in info.cache_key
    assert info.cache_key.endswith("_0") and " " not in info.cache_key
    assert info.clock_mhz and info.clock_mhz > 500
    assert info.driver_version


def test_public_api_on_gpu_passes_the_gate() -> None:
    x = _rand(4, 256, 4096, dtype=torch.float16)
    r = _rand(4, 256, 4096, dtype=torch.float16, seed=2)
    w = _rand(4096, dtype=torch.float16, seed=1, scale=0.1, shift=1.0)
    ref = rmsnorm_ref(x, w)
    assert max_abs_error(ref, ako_amd.rmsnorm(x, w)) <= error_budget(ref)
    got = ako_amd.rmsnorm_residual(x, r, w)
    ref2 = (rmsnorm_ref(x + r, w), x + r)
    assert max_abs_error_any(ref2, got) <= error_budget(ref2)
    q = _rand(2, 64, 32, 128)
    cos, sin = build_rope_tables(64, 128, device=DEV)
    qo, ko = ako_amd.rope_qk(q, q, cos, sin)
    ref3 = rope_ref(q, cos, sin)
    assert max_abs_error(ref3, qo) <= error_budget(ref3) and torch.equal(qo, ko)
    g, u = _rand(8, 14336), _rand(8, 14336, seed=3)
    out = ako_amd.swiglu(g, u, kernel="swiglu_hip")
    assert out.shape == g.shape


def test_hip_graph_replays_match_eager() -> None:
    """Every HIP kernel captured in one graph; each replay (with eager work and
    synchronisation in between) must equal the eager result bit for bit."""
    x = _rand(32, 4096)
    r = _rand(32, 4096, seed=1)
    w = _rand(4096, seed=2, scale=0.1, shift=1.0)
    q = _rand(1, 1, 32, 128, seed=3)
    k = _rand(1, 1, 8, 128, seed=4)
    cos, sin = build_rope_tables(1, 128, device=DEV)
    g, u = _rand(1, 14336, seed=5), _rand(1, 14336, seed=6)
    # Launches of many rows: the persistent pipelined kernel (4096-wide rows)
    # and bf16 residual rows of 16384 with one-packet load groups.
    xp, rp = _rand(9000, 4096, seed=7), _rand(9000, 4096, seed=8)
    xb, rb = _rand(300, 16384, seed=9), _rand(300, 16384, seed=10)
    wb = _rand(16384, seed=11, scale=0.1, shift=1.0)

    def step():
        a = rmsnorm_hip(x, w)
        b, c = rmsnorm_residual_hip(x, r, w)
        d = rope_hip(q, cos, sin)
        e, f = rope_qk_hip(q, k, cos, sin, "interleaved")
        h = swiglu_hip(g, u)
        i = rmsnorm_hip(xp, w)
        j, m = rmsnorm_residual_hip(xp, rp, w)
        n, o = rmsnorm_residual_hip(xb, rb, wb)
        return a, b, c, d, e, f, h, i, j, m, n, o

    eager = step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for i in range(4):
        for t in captured:
            t.zero_()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for want, got in zip(eager, captured):
            assert torch.equal(want, got), f"replay {i} differs"


def test_cache_rope_graph_follows_the_device_position() -> None:
    """rope_qk_cache captured once with the position advanced inside the graph:
    replay n writes slot start + n, exactly as the eager call at that position."""
    hq, hkv, d, cache_len, start = 8, 2, 128, 24, 5
    q = _rand(1, 1, hq, d, dtype=torch.float16, seed=7)
    k = _rand(1, 1, hkv, d, dtype=torch.float16, seed=8)
    v = _rand(1, 1, hkv, d, dtype=torch.float16, seed=9)
    cos, sin = build_rope_tables(cache_len, d, device=DEV)
    kc = torch.zeros(1, hkv, cache_len, d, device=DEV, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    pos = torch.full((1,), start, dtype=torch.int64, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        rope_qk_cache_hip(q, k, v, cos, sin, pos, kc, vc)  # warm-up, rewritten by replay 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        q_out = rope_qk_cache_hip(q, k, v, cos, sin, pos, kc, vc)
        pos.add_(1)
    kc_eager, vc_eager = torch.zeros_like(kc), torch.zeros_like(vc)
    for n in range(6):
        for t, seed in ((q, 20 + n), (k, 30 + n), (v, 40 + n)):  # new token, eager work between replays
            t.copy_(_rand(*t.shape, dtype=t.dtype, seed=seed))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        at = torch.tensor([start + n], dtype=torch.int64, device=DEV)
        want_q = rope_qk_cache_hip(q, k, v, cos, sin, at, kc_eager, vc_eager)
        assert torch.equal(q_out, want_q), n
        assert int(pos.item()) == start + n + 1
    assert torch.equal(kc, kc_eager) and torch.equal(vc, vc_eager)
    assert not kc[:, :, :start].any() and not kc[:, :, start + 6:].any()


@pytest.mark.parametrize("n_kv_heads", [4, 2])
def test_decoder_backends_agree_on_gpu(n_kv_heads: int) -> None:
    from ako_amd.models.decoder import ModelConfig, build_lm

    cfg = ModelConfig(hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=n_kv_heads, intermediate_dim=1024,
                      max_seq_len=96, vocab_size=1000, eps=1e-6)
    prompt = torch.randint(0, 1000, (1, 33), generator=torch.Generator().manual_seed(0)).to(DEV)
    outs = {}
    for backend in ("torch", "ako"):
        model = build_lm(cfg, backend=backend, device=DEV, dtype=torch.float16, seed=3)
        cache = model.stack.new_kv_cache(64)
        with torch.no_grad():
            outs[backend] = model.logits_last(prompt, cache).float()
            outs[backend + "_dec"] = model.logits_last(prompt[:, :1], cache).float()
    for key in ("", "_dec"):
        a, b = outs["ako" + key], outs["torch" + key]
        assert (a - b).abs().max().item() <= 2e-2 * b.abs().max().item() + 1e-3


@pytest.mark.parametrize("n_kv_heads", [4, 2])
def test_graphed_greedy_matches_eager_static_decoding(n_kv_heads: int) -> None:
    from ako_amd.models.decoder import GraphedGreedy, ModelConfig, build_lm

    cfg = ModelConfig(hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=n_kv_heads, intermediate_dim=1024,
                      max_seq_len=64, vocab_size=1000, eps=1e-6)
    prompt = torch.randint(0, 1000, (1, 17), generator=torch.Generator().manual_seed(1)).to(DEV)
    for backend in ("ako", "torch"):
        model = build_lm(cfg, backend=backend, device=DEV, dtype=torch.float16, seed=4)
        with torch.no_grad():
            cache = model.stack.new_static_cache(17 + 12)
            ids = model.logits_last(prompt, cache).argmax(-1, keepdim=True)
            eager = [ids]
            for _ in range(11):
                ids = model.logits_last(ids, cache).argmax(-1, keepdim=True)
                eager.append(ids)
            eager_tokens = torch.cat(eager, 1)
            for _ in range(2):  # two independent runners: every replay must reproduce eager
                runner = GraphedGreedy(model, prompt, 12)
                graphed = runner.run()
                torch.cuda.synchronize()
                assert torch.equal(graphed, eager_tokens), (backend, graphed, eager_tokens)
                assert runner.cache.length == 17 + 11
                with pytest.raises(RuntimeError, match="decodes once"):
                    runner.run()  # a second pass would step past the slab


def test_torch_binding_matches_the_ctypes_path() -> None:
    """The C++ binding and the ctypes path launch the same kernels: identical
    outputs, the same errors, and torch's current stream (side streams too)."""
    from ako_amd import _native
    from ako_amd.ops import rmsnorm_hip as rm, rope_hip as rp, swiglu_hip as sw

    fast = _native.torch_binding()
    assert fast is not None
    x, r = _rand(33, 4096, seed=40), _rand(33, 4096, seed=41)
    w = _rand(4096, seed=42, scale=0.1, shift=1.0)
    q, k, v = _rand(2, 5, 8, 128, seed=43), _rand(2, 5, 2, 128, seed=44), _rand(2, 5, 2, 128, seed=45)
    cos, sin = build_rope_tables(16, 128, device=DEV)
    g, u = _rand(7, 1000, seed=46), _rand(7, 1000, seed=47)
    assert torch.equal(fast.rmsnorm(x, w, 1e-6), rm.rmsnorm_hip_ctypes(x, w, 1e-6))
    for a, b in zip(fast.rmsnorm_residual(x, r, w, 1e-6), rm.rmsnorm_residual_hip_ctypes(x, r, w, 1e-6)):
        assert torch.equal(a, b)
    assert torch.equal(fast.rope(q, cos[:5], sin[:5], "interleaved"), rp.rope_hip_ctypes(q, cos[:5], sin[:5], "interleaved"))
    for a, b in zip(fast.rope_qk(q, k, cos[:5], sin[:5], "neox"), rp.rope_qk_hip_ctypes(q, k, cos[:5], sin[:5], "neox")):
        assert torch.equal(a, b)
    pos = torch.full((1,), 3, dtype=torch.long, device=DEV)
    caches = [torch.zeros(2, 2, 16, 128, device=DEV, dtype=torch.bfloat16) for _ in range(4)]
    qa = fast.rope_qk_cache(q, k, v, cos, sin, pos, caches[0], caches[1], "neox")
    qb = rp.rope_qk_cache_hip_ctypes(q, k, v, cos, sin, pos, caches[2], caches[3], "neox")
    assert torch.equal(qa, qb) and torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    assert torch.equal(fast.swiglu(g, u), sw.swiglu_hip_ctypes(g, u))
    bad = [
        (lambda: fast.rmsnorm(x, w[:100], 1e-6), lambda: rm.rmsnorm_hip_ctypes(x, w[:100], 1e-6)),
        (lambda: fast.rope(q, cos, sin, "neox"), lambda: rp.rope_hip_ctypes(q, cos, sin, "neox")),
        (lambda: fast.rope(q, cos[:5], sin[:5], "rot"), lambda: rp.rope_hip_ctypes(q, cos[:5], sin[:5], "rot")),
        (lambda: fast.rope_qk_cache(q, k, v, cos, sin, pos.int(), caches[0], caches[1], "neox"),
         lambda: rp.rope_qk_cache_hip_ctypes(q, k, v, cos, sin, pos.int(), caches[0], caches[1], "neox")),
        (lambda: fast.swiglu(g, u[:3]), lambda: sw.swiglu_hip_ctypes(g, u[:3])),
    ]
    for fast_call, slow_call in bad:
        with pytest.raises(ValueError) as ea:
            fast_call()
        with pytest.raises(ValueError) as eb:
            slow_call()
        assert str(ea.value) == str(eb.value)
    assert fast.current_stream(0) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert fast.current_stream(0) == side.cuda_stream
        y_side = fast.rmsnorm(x, w, 1e-6)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(y_side, rm.rmsnorm_hip_ctypes(x, w, 1e-6))


@pytest.mark.parametrize("fused_qkv", [True, False])
@pytest.mark.parametrize("n_kv_heads", [4, 2])
def test_stack_on_hip_kernels_matches_hugging_face_llama(n_kv_heads: int, fused_qkv: bool) -> None:
    """The decoder with the HIP kernels (fp32) against Hugging Face's LlamaModel
    carrying the same weights, prompt and cached decoding, on the GPU. With the
    fused projection q, k and v reach the RoPE kernels as strided column
    slices of one GEMM output; without it, as contiguous tensors."""
    from tests.test_model import _hf_pair

    hf, stacks = _hf_pair(n_kv_heads, fused_qkv)
    hf, stack = hf.to(DEV), stacks["ako"].to(DEV)
    ids = torch.randint(0, 50, (1, 12), generator=torch.Generator().manual_seed(2)).to(DEV)
    with torch.no_grad():
        want = hf(input_ids=ids).last_hidden_state
        emb = hf.embed_tokens(ids)
        torch.testing.assert_close(stack(emb), want, atol=2e-5, rtol=2e-5)
        for cache in (stack.new_kv_cache(16), stack.new_static_cache(16)):
            got = [stack(emb[:, :9], kv_cache=cache)[:, -1]]
            for t in range(9, 12):
                got.append(stack(emb[:, t:t + 1], kv_cache=cache)[:, -1])
            torch.testing.assert_close(torch.stack(got, 1), want[:, 8:12], atol=2e-5, rtol=2e-5)


def test_config5_workload_selection(tmp_path) -> None:
    """The offline selection for the configs[4] decoder's shapes (prefill of
    512 tokens and a decode step): every decision passes the gate, and the HIP
    candidate is chosen for (nearly) every operation."""
    from ako_amd.benchmark.optimize import config5_phases, optimize

    doc = optimize(config5_phases(), device=torch.device(DEV), cache=KernelCache(path=tmp_path / "c.json"),
                   warmup=3, repeats=10)
    ops = doc["operations"]
    assert len(ops) == 10 and "decode/rope_qk" in ops and "prefill/swiglu" in ops
    hip = [name for name, op in ops.items() if op["backend"] == "hip"]
    print({name: (op["selected_kernel"], op["speedup_vs_best_baseline"]) for name, op in ops.items()})
    for op in ops.values():
        assert op["source"] == "benchmark" and all(r["passed"] for r in op["ulp_reports"] if r["kernel"].endswith("_hip"))
    assert len(hip) >= 9, hip


def test_minimal_reference_side_binding() -> None:
    """The least a maintainer of the reference would write to bind the C ABI
    (a fresh ctypes handle, the declared argument types, raw pointers and the
    current stream): the same bits as this package's wrapper, and the status
    and message contract on a bad argument."""
    import ctypes

    from ako_amd._native import library_path

    lib = ctypes.CDLL(str(library_path()))
    lib.ako_rmsnorm_fwd.restype = ctypes.c_int
    lib.ako_rmsnorm_fwd.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 4 + \
        [ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.ako_last_error.restype = ctypes.c_char_p
    codes = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

    def rmsnorm_minimal(x, weight, eps=1e-6):
        h = x.shape[-1]
        x2 = x.contiguous()
        y = torch.empty_like(x2)
        rc = lib.ako_rmsnorm_fwd(x2.data_ptr(), weight.contiguous().data_ptr(), y.data_ptr(),
                                 x2.numel() // h, h, h, h, eps, codes[x.dtype], codes[weight.dtype],
                                 torch.cuda.current_stream().cuda_stream)
        if rc:
            raise (ValueError if rc in (1, 2) else RuntimeError)(lib.ako_last_error().decode())
        return y.view(x.shape)

    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        x = _rand(3, 700, 4096, dtype=dtype, seed=80)
        w = _rand(4096, dtype=dtype, seed=81, scale=0.1, shift=1.0)
        assert torch.equal(rmsnorm_minimal(x, w), rmsnorm_hip(x, w, 1e-6))
        w32 = w.float()
        assert torch.equal(rmsnorm_minimal(x, w32), rmsnorm_hip(x, w32, 1e-6))
    with pytest.raises(ValueError, match="eps"):
        rmsnorm_minimal(x, w, -1.0)

