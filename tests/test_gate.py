"""The dtype-aware gate (ako_amd.validation.numerical), behaviour of the
reference's tests/test_tolerance.py:21-125 on this package."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.registry import KernelEntry, KernelRegistry
from ako_amd.dispatcher.selector import KernelSelector
from ako_amd.ops.rmsnorm_ref import rmsnorm_ref
from ako_amd.validation.numerical import (
    DTYPE_RTOL,
    error_budget,
    error_in_ulps,
    max_abs_error,
    max_abs_error_any,
    ulp,
    ulp_report,
)

REF = json.loads((Path(__file__).resolve().parent / "golden" / "reference_golden.json").read_text())
DT = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def test_ulp_known_answers() -> None:
    for dtype, magnitude, expected in REF["ulp_known_answers"]["cases"]:
        assert ulp(DT[dtype], magnitude) == pytest.approx(expected)
    assert ulp(torch.bfloat16, 0.0) > 0
    # Exact at binade edges (2**k and just below it).
    assert ulp(torch.float16, 4.0) == 2.0**2 * 2.0**-10
    assert ulp(torch.float16, 3.9999) == 2.0**1 * 2.0**-10


def test_rtol_table_is_the_reference_table() -> None:
    assert DTYPE_RTOL == {torch.float64: 1e-7, torch.float32: 1.3e-6,
                          torch.float16: 1e-3, torch.bfloat16: 1.6e-2}


def test_bf16_rounding_alone_exceeds_a_flat_1e_2() -> None:
    exact = torch.randn(4096, generator=torch.Generator().manual_seed(0)) * 5.0
    rounded = exact.to(torch.bfloat16)
    err = max_abs_error(exact, rounded.float())
    assert err > 1e-2
    assert err <= ulp(torch.bfloat16, exact.abs().max().item()) / 2
    assert err < error_budget(rounded)


def test_budget_scales_with_dtype_and_magnitude() -> None:
    g = torch.Generator().manual_seed(1)
    small = (torch.randn(128, generator=g) * 0.01).to(torch.bfloat16)
    large = (torch.randn(128, generator=g) * 100.0).to(torch.bfloat16)
    assert error_budget(large) > error_budget(small)
    values = torch.randn(128, generator=g) * 5.0
    assert error_budget(values) < error_budget(values.half()) < error_budget(values.bfloat16())
    assert error_budget(values, tol_scale=2.0) == pytest.approx(2 * error_budget(values))


def test_budget_and_error_accept_tuples() -> None:
    a = torch.randn(64).to(torch.bfloat16)
    b = (torch.randn(64) * 50.0).to(torch.bfloat16)
    assert error_budget((a, b)) == error_budget(b)
    assert max_abs_error_any((a, b), (a, b)) == 0.0
    with pytest.raises(ValueError):
        max_abs_error_any((a, b), (a,))
    with pytest.raises(TypeError):
        max_abs_error_any(a, [a])


def test_error_in_ulps_is_dtype_independent() -> None:
    for dtype in (torch.float16, torch.bfloat16):
        reference = (torch.randn(256, generator=torch.Generator().manual_seed(2)) * 5.0).to(dtype)
        spacing = ulp(dtype, reference.float().abs().max().item())
        shifted = (reference.float() + spacing).to(dtype)
        assert error_in_ulps(reference, shifted) == pytest.approx(1.0, rel=0.3)


def test_ulp_report_fields() -> None:
    ref = torch.tensor([1.0, -3.0, 2.5], dtype=torch.float16)
    rep = ulp_report(ref, ref, kernel="k")
    assert rep["passed"] and rep["err_ulps"] == 0.0 and rep["kernel"] == "k"
    assert rep["budget_ulps"] == pytest.approx(rep["error_budget"] / rep["ulp"])


def _selector(candidate, tmp_path, **kwargs) -> KernelSelector:
    reg = KernelRegistry()
    reg.register(KernelEntry("rmsnorm", "rmsnorm_ref", rmsnorm_ref, backend="pytorch", priority=10))
    reg.register(KernelEntry("rmsnorm", "candidate", candidate, backend="hip", priority=5))
    return KernelSelector(registry=reg, cache=KernelCache(path=tmp_path / "c.json"), warmup=1,
                          repeats=3, allow_cpu_tuning=True, **kwargs)


def _one_ulp_off(x, weight, eps=1e-6):
    out = rmsnorm_ref(x, weight, eps).float()
    return (out + ulp(torch.bfloat16, out.abs().max().item())).to(x.dtype)


def _inputs():
    g = torch.Generator().manual_seed(3)
    return (torch.randn(64, 512, generator=g) * 5.0).to(torch.bfloat16), torch.ones(512, dtype=torch.bfloat16)


def test_flat_threshold_rejects_a_correct_bf16_kernel(tmp_path) -> None:
    result = _selector(_one_ulp_off, tmp_path, error_threshold=1e-2).select_entry("rmsnorm", *_inputs())
    assert result.entry.kernel_name == "rmsnorm_ref"
    assert any("candidate" in r for r in result.rejected)


def test_dtype_budget_keeps_a_correct_bf16_kernel(tmp_path) -> None:
    result = _selector(_one_ulp_off, tmp_path).select_entry("rmsnorm", *_inputs())
    assert result.rejected == ()
    assert result.candidates_evaluated == 2
    assert result.ulp_reports[0]["passed"] and result.ulp_reports[0]["err_ulps"] <= 1.5


def test_budget_rejects_a_wrong_kernel_with_ulps(tmp_path) -> None:
    result = _selector(lambda x, w, eps=1e-6: torch.zeros_like(x), tmp_path).select_entry("rmsnorm", *_inputs())
    assert result.entry.kernel_name == "rmsnorm_ref"
    assert any("ulps" in r for r in result.rejected)
    assert result.ulp_reports[0]["passed"] is False


def test_reference_rejection_line_reproduced(tmp_path) -> None:
    """docs/EXTENDING.md:153-175 of the reference, through this selector."""
    gold = REF["extending_rejection"]

    def rmsnorm_wrong(x, weight, eps=1e-6):
        xc = x.float()
        return (xc * torch.rsqrt(xc.abs().mean(dim=-1, keepdim=True) + eps) * weight.float()).to(x.dtype)

    torch.manual_seed(0)
    x = torch.randn(4096, 2048)
    weight = torch.randn(2048)
    reg = KernelRegistry()
    reg.register(KernelEntry("rmsnorm", "rmsnorm_ref", rmsnorm_ref, backend="pytorch", priority=10))
    reg.register(KernelEntry("rmsnorm", "rmsnorm_wrong", rmsnorm_wrong, backend="custom", priority=1))
    sel = KernelSelector(registry=reg, cache=KernelCache(path=tmp_path / "c.json"),
                         allow_cpu_tuning=True, warmup=1, repeats=2)
    result = sel.select_entry("rmsnorm", x, weight)
    expected = (f"rmsnorm_wrong: max_error={gold['max_error']} > budget={gold['budget']} "
                f"({gold['ulps']} ulps)")
    assert result.rejected == (expected,)
