"""BASELINE.json configs[4] on the GPU at its own size.

A 4-layer Llama-style decoder (hidden 4096, 32 heads x 128, FFN 11008, RMSNorm
eps 1e-6, RoPE theta 1e4, fp16, N(0, 0.02) init, vocab 32000, batch 1) built
twice from one seed: ``backend="ako"`` sends norm/rope/swiglu through the
dispatcher (the HIP candidates win there), ``backend="torch"`` runs the
reference's unfused eager path (``ako/models/decoder.py:101-216``). GEMMs and
attention are PyTorch-ROCm in both.

* A third copy, ``hip``, is the ako backend with every dispatched op forced
  to its HIP candidate (the reference decoder's per-op ``KernelOverride``,
  ``ako/models/decoder.py:101-134``): the numerical checks below run on it as
  on the selected ``ako`` copy, so they hold for the HIP kernels whatever the
  selector picks, and the selector's decisions are recorded to show which
  candidate each dispatched call ran.
* The truth is a fourth copy: the torch backend in fp32 with the same
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
#: Every dispatched op of the decoder forced to its HIP candidate.
FORCE_HIP = {"rmsnorm": "rmsnorm_hip", "rmsnorm_residual": "rmsnorm_residual_hip",
             "rope_qk": "rope_qk_hip", "swiglu": "swiglu_hip"}
DISPATCHED = set(FORCE_HIP)


@pytest.fixture(scope="module")
def models():
    import copy

    cfg = dec.config5()
    cfg.max_seq_len = PROMPT + STEPS
    built = {b: dec.build_lm(cfg, backend=b, device=DEV, dtype=torch.float16, seed=0)
             for b in ("torch", "ako")}
    built["hip"] = dec.build_lm(cfg, backend="ako", device=DEV, dtype=torch.float16, seed=0,
                                kernel_override=FORCE_HIP)
    built["fp32"] = copy.deepcopy(built["torch"]).float()
    prompt = torch.randint(0, cfg.vocab_size, (1, PROMPT), generator=torch.Generator().manual_seed(0)).to(DEV)
    yield cfg, built, prompt
    del built
    torch.cuda.empty_cache()


def _errors(logits: dict[str, torch.Tensor], which: str = "ako") -> tuple[float, float, float]:
    """(dispatched error, native fp16 error) against the fp32 run, and the
    fp16 gate budget of the fp32 logits; ``which`` names the dispatched copy."""
    ref = logits["fp32"].float()
    err_a = (logits[which].float() - ref).abs().max().item()
    err_t = (logits["torch"].float() - ref).abs().max().item()
    return err_a, err_t, error_budget(ref.half())


@pytest.fixture
def decisions(monkeypatch):
    """Every selection made while the test runs: ``(op, kernel, backend,
    source)``, with the selector's per-call memo emptied first so that each
    call site's first call is seen."""
    from ako_amd.dispatcher import selector as sel

    sel.reset_selector()
    seen: list[tuple[str, str, str, str]] = []
    original = sel.KernelSelector.select_entry

    def recording(self, op_name, *args, **kwargs):
        result = original(self, op_name, *args, **kwargs)
        seen.append((op_name, result.entry.kernel_name, result.entry.backend, result.source))
        return result

    monkeypatch.setattr(sel.KernelSelector, "select_entry", recording)
    yield seen
    sel.reset_selector()


def test_config5_geometry(models) -> None:
    cfg, built, _ = models
    assert (cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.head_dim, cfg.intermediate_dim) == (4096, 4, 32, 128, 11008)
    assert (cfg.eps, cfg.rope_base, cfg.vocab_size) == (1e-6, 10000.0, 32000)
    p = next(built["ako"].parameters())
    assert p.dtype == torch.float16 and p.is_cuda
    # Same seed, same weights in every copy.
    for (na, a), (nt, t), (nh, h), (nf, f) in zip(
            built["ako"].named_parameters(), built["torch"].named_parameters(),
            built["hip"].named_parameters(), built["fp32"].named_parameters()):
        assert na == nt == nh == nf and torch.equal(a, t) and torch.equal(a, h) and torch.equal(a.float(), f), na


def test_config5_prefill_and_teacher_forced_decode(models, decisions, monkeypatch) -> None:
    _, built, prompt = models
    # The selected copy rotates q/k with rope_qk_cache on its preallocated
    # cache: a direct call of the HIP entry point, not a dispatched op.
    fused_calls = []
    direct = dec.rope_qk_cache

    def counting(*args, **kwargs):
        fused_calls.append(args[0].shape[1])
        return direct(*args, **kwargs)

    monkeypatch.setattr(dec, "rope_qk_cache", counting)
    caches = {b: m.stack.new_kv_cache(PROMPT + STEPS) for b, m in built.items()}
    dispatched = ("ako", "hip")
    with torch.no_grad():
        logits = {b: built[b].logits_last(prompt, caches[b]) for b in built}
        for which in dispatched:
            err_a, err_t, budget = _errors(logits, which)
            print(f"config5 prefill vs fp32: {which} {err_a:.3e}, torch fp16 {err_t:.3e}, "
                  f"gate budget {budget:.3e}", flush=True)
            assert err_a <= max(2 * err_t, budget), (which, err_a, err_t, budget)
        worst = dict.fromkeys(dispatched, 0.0)
        checked = dict.fromkeys(dispatched, 0)
        agreed = dict.fromkeys(dispatched, 0)
        for step in range(STEPS):
            top2 = logits["fp32"].topk(2, dim=-1).values[0]
            margin = (top2[0] - top2[1]).item()
            truth = logits["fp32"].argmax(-1)
            for which in dispatched:
                err_a, err_t, budget = _errors(logits, which)
                bar = max(2 * err_t, budget)
                worst[which] = max(worst[which], err_a / bar)
                assert err_a <= bar, (f"step {step}: {which} {err_a:.3e} > max(2 x torch {err_t:.3e}, "
                                      f"{budget:.3e})")
                a_tok = logits[which].argmax(-1)
                if margin > 2 * err_a:
                    checked[which] += 1
                    assert torch.equal(a_tok, truth), f"step {step}: margin {margin:.3e}, {which} token differs"
                agreed[which] += int(torch.equal(a_tok, truth))
            if step + 1 == STEPS:
                break
            nxt = truth.view(1, 1)  # teacher forcing: every copy sees the fp32 token
            logits = {b: built[b].logits_last(nxt, caches[b]) for b in built}
    for which in dispatched:
        print(f"config5 decode ({which}): {STEPS} steps, worst error / bar {worst[which]:.3f}, argmax checked "
              f"on {checked[which]}, equal on {agreed[which]}", flush=True)
        assert checked[which] >= STEPS // 2  # the margin rule must leave most steps checked
    # What ran: the forced copy's calls are all the HIP entries; the selected
    # copy's decisions are printed, and HIP must hold at least 90% of them.
    forced = [d for d in decisions if d[3] == "forced"]
    chosen = [d for d in decisions if d[3] != "forced"]
    assert {d[0] for d in forced} == DISPATCHED, forced
    assert all(d[1] == FORCE_HIP[d[0]] and d[2] == "hip" for d in forced), forced
    assert {d[0] for d in chosen} == DISPATCHED - {"rope_qk"}, chosen
    assert len(fused_calls) == 4 * STEPS and fused_calls[0] == PROMPT, fused_calls[:8]
    hip = sum(d[2] == "hip" for d in chosen)
    print(f"config5 selected copy: {hip} of {len(chosen)} decisions chose HIP; others: "
          f"{sorted({d for d in chosen if d[2] != 'hip'})}", flush=True)
    assert hip >= 0.9 * len(chosen), chosen


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


@pytest.mark.parametrize("which", ["hip", "ako"])
def test_config5_layer0_kernels_against_the_oracle(models, monkeypatch, which) -> None:
    """The dispatched calls of layer 0 at prefill, recorded as the model runs,
    against the oracle on 64 sampled token rows (rows are independent): on
    the copy forced to the HIP candidates and on the selected copy."""
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
        built[which].logits_last(prompt, built[which].stack.new_kv_cache())
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
