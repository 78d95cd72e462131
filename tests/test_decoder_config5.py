"""BASELINE.json configs[4] on the GPU at its own size.

A 4-layer Llama-style decoder (hidden 4096, 32 heads x 128, FFN 11008, RMSNorm
eps 1e-6, RoPE theta 1e4, fp16, N(0, 0.02) init, vocab 32000, batch 1) built
twice from one seed: ``backend="ako"`` sends norm/rope/swiglu through the
dispatcher (the HIP candidates win there), ``backend="torch"`` runs the
reference's unfused eager path (``ako/models/decoder.py:101-216``). GEMMs and
attention are PyTorch-ROCm in both.

* The truth is a third copy: the torch backend in fp32 with the same
  (fp16-rounded) weights. The single-op gate (``atol + rtol(fp16)*max|ref|``,
  about one fp16 ulp of the largest logit) is the bar for one kernel's output;
  four layers of fp16 GEMMs and the reference's own ``F.silu(g) * up`` (two
  roundings) move the fp16 eager path's logits by more than that. So, as the
  reference's ``tests/test_numerical_bounds.py:153-180`` does for single ops,
  the dispatched path must stay within 2x the native fp16 path's error against
  the fp32 run (never held below the fp16 gate budget).
* Prefill of 512 seeded token ids: that rule on the last-position logits.
* 128 greedy steps, teacher-forced with the fp32 run's tokens so that one
  near-tie cannot send the runs down different continuations: the same rule on
  every step's logits, and the dispatched path's argmax equals the fp32 argmax
  wherever the fp32 top-2 margin exceeds twice its measured error.
* Graph-replayed greedy decoding (``GraphedGreedy``) gives the tokens of eager
  decoding through the same static cache.
* Layer 0's dispatched RMSNorm, residual RMSNorm, RoPE and SwiGLU outputs at
  prefill are checked against the CPU oracle on sampled rows.

Mirrors the reference's ``tests/test_model.py:21-79`` (backends agree, KV
decode) at the configs[4] size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ako_amd.models import decoder as dec
from ako_amd.validation.numerical import error_budget
from oracle import ops as oracle
from tests._util import to_np

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"
PROMPT, STEPS = 512, 128


@pytest.fixture(scope="module")
def models():
    import copy

    cfg = dec.config5()
    cfg.max_seq_len = PROMPT + STEPS
    built = {b: dec.build_lm(cfg, backend=b, device=DEV, dtype=torch.float16, seed=0)
             for b in ("torch", "ako")}
    built["fp32"] = copy.deepcopy(built["torch"]).float()
    prompt = torch.randint(0, cfg.vocab_size, (1, PROMPT), generator=torch.Generator().manual_seed(0)).to(DEV)
    yield cfg, built, prompt
    del built
    torch.cuda.empty_cache()


def _errors(logits: dict[str, torch.Tensor]) -> tuple[float, float, float]:
    """(dispatched error, native fp16 error) against the fp32 run, and the
    fp16 gate budget of the fp32 logits."""
    ref = logits["fp32"].float()
    err_a = (logits["ako"].float() - ref).abs().max().item()
    err_t = (logits["torch"].float() - ref).abs().max().item()
    return err_a, err_t, error_budget(ref.half())


def test_config5_geometry(models) -> None:
    cfg, built, _ = models
    assert (cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.head_dim, cfg.intermediate_dim) == (4096, 4, 32, 128, 11008)
    assert (cfg.eps, cfg.rope_base, cfg.vocab_size) == (1e-6, 10000.0, 32000)
    p = next(built["ako"].parameters())
    assert p.dtype == torch.float16 and p.is_cuda
    # Same seed, same weights in every copy.
    for (na, a), (nt, t), (nf, f) in zip(built["ako"].named_parameters(), built["torch"].named_parameters(),
                                         built["fp32"].named_parameters()):
        assert na == nt == nf and torch.equal(a, t) and torch.equal(a.float(), f), na


def test_config5_prefill_and_teacher_forced_decode(models) -> None:
    _, built, prompt = models
    caches = {b: m.stack.new_kv_cache(PROMPT + STEPS) for b, m in built.items()}
    with torch.no_grad():
        logits = {b: built[b].logits_last(prompt, caches[b]) for b in built}
        err_a, err_t, budget = _errors(logits)
        print(f"config5 prefill vs fp32: ako {err_a:.3e}, torch fp16 {err_t:.3e}, gate budget {budget:.3e}",
              flush=True)
        assert err_a <= max(2 * err_t, budget), (err_a, err_t, budget)
        worst, checked, agreed = 0.0, 0, 0
        for step in range(STEPS):
            err_a, err_t, budget = _errors(logits)
            bar = max(2 * err_t, budget)
            worst = max(worst, err_a / bar)
            assert err_a <= bar, f"step {step}: ako {err_a:.3e} > max(2 x torch {err_t:.3e}, {budget:.3e})"
            top2 = logits["fp32"].topk(2, dim=-1).values[0]
            margin = (top2[0] - top2[1]).item()
            truth = logits["fp32"].argmax(-1)
            a_tok = logits["ako"].argmax(-1)
            if margin > 2 * err_a:
                checked += 1
                assert torch.equal(a_tok, truth), f"step {step}: margin {margin:.3e}, ako token differs"
            agreed += int(torch.equal(a_tok, truth))
            if step + 1 == STEPS:
                break
            nxt = truth.view(1, 1)  # teacher forcing: every copy sees the fp32 token
            logits = {b: built[b].logits_last(nxt, caches[b]) for b in built}
    print(f"config5 decode: {STEPS} steps, worst error / bar {worst:.3f}, argmax checked on {checked}, "
          f"equal on {agreed}", flush=True)
    assert checked >= STEPS // 2  # the margin rule must leave most steps checked


def test_config5_graphed_decode_matches_eager(models) -> None:
    _, built, prompt = models
    model = built["ako"]
    with torch.no_grad():
        cache = model.stack.new_static_cache(PROMPT + STEPS)
        ids = model.logits_last(prompt, cache).argmax(-1, keepdim=True)
        eager = [ids]
        for _ in range(STEPS - 1):
            ids = model.logits_last(ids, cache).argmax(-1, keepdim=True)
            eager.append(ids)
        eager_tokens = torch.cat(eager, 1)
        graphed = dec.GraphedGreedy(model, prompt, STEPS).run()
        torch.cuda.synchronize()
    assert torch.equal(graphed, eager_tokens)


def test_config5_layer0_kernels_against_the_oracle(models, monkeypatch) -> None:
    """The dispatched calls of layer 0 at prefill, recorded as the model runs,
    against the oracle on 64 sampled token rows (rows are independent)."""
    _, built, prompt = models
    seen: dict[str, tuple] = {}

    def record(name, fn):
        def wrapped(*args, **kwargs):
            out = fn(*args, **kwargs)
            seen.setdefault(name, (args, out))
            return out
        return wrapped

    for name in ("rmsnorm", "rmsnorm_residual", "rope_qk", "swiglu"):
        monkeypatch.setattr(dec, name, record(name, getattr(dec, name)))
    with torch.no_grad():
        # A growing cache (no slab): prefill rotates q and k with rope_qk.
        built["ako"].logits_last(prompt, built["ako"].stack.new_kv_cache())
    torch.cuda.synchronize()
    assert set(seen) == {"rmsnorm", "rmsnorm_residual", "rope_qk", "swiglu"}, set(seen)
    rows = np.unique(np.concatenate([[0, PROMPT - 1],
                                     np.random.default_rng(5).choice(PROMPT, 62, replace=False)]))
    sel = torch.as_tensor(rows, device=DEV)

    def assert_close(expected, got):
        rep = oracle.gate(expected, got, "float16")
        assert rep["passed"] and rep["err_ulps"] <= 2.0, rep

    (x, w, eps), y = seen["rmsnorm"][0][:3], seen["rmsnorm"][1]
    assert x.shape == (1, PROMPT, 4096)
    assert_close(oracle.rmsnorm(to_np(x[0, sel]), to_np(w), eps, dtype="float16"), to_np(y[0, sel]))
    (x, r, w, eps), (y, s) = seen["rmsnorm_residual"][0][:4], seen["rmsnorm_residual"][1]
    ey, es = oracle.rmsnorm_residual(to_np(x[0, sel]), to_np(r[0, sel]), to_np(w), eps, dtype="float16")
    np.testing.assert_array_equal(to_np(s[0, sel]), es)
    assert_close(ey, to_np(y[0, sel]))
    (q, k, cos, sin), (qo, ko) = seen["rope_qk"][0][:4], seen["rope_qk"][1]
    assert q.shape == (1, PROMPT, 32, 128) and cos.shape == (PROMPT, 64)
    for src, out in ((q, qo), (k, ko)):
        exp = oracle.rope(to_np(src[:, sel]), to_np(cos[sel]), to_np(sin[sel]), "neox", dtype="float16")
        np.testing.assert_array_equal(to_np(out[:, sel]), exp)  # RoPE is bit-exact
    (g, u), y = seen["swiglu"][0][:2], seen["swiglu"][1]
    assert g.shape == (1, PROMPT, 11008)
    assert_close(oracle.swiglu(to_np(g[0, sel]), to_np(u[0, sel]), dtype="float16"), to_np(y[0, sel]))
