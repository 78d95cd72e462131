"""The numerical gate: dtype- and magnitude-scaled error budgets, ulp accounting.

Follows ``ako/validation/numerical.py:20-122`` of the reference unchanged in
behaviour: a candidate output is accepted when

    max |ref - cand|  <=  tol_scale * (atol + rtol(dtype) * max |ref|)

with ``rtol`` taken per dtype (the ``torch.testing.assert_close`` defaults) and
``atol = 1e-5``. Tuple outputs (``rmsnorm_residual`` returns two tensors) are
compared item by item; their magnitude is the largest over items and their
dtype is the dtype of the first item (reference ``numerical.py:68-74``).

A flat absolute threshold cannot work across dtypes: around magnitude 5 two
neighbouring bf16 values are 2**-5 = 0.031 apart, so two correct kernels that
round differently already disagree by more than 1e-2.

``ulp_report`` is new: it packages the per-candidate numbers the MI355X build
reports (max error, budget, error in ulps at ``max|ref|``, pass/fail).
"""

from __future__ import annotations

import math
from typing import Any, Sequence

import torch

#: Allowed relative spacing between two correct implementations, per dtype
#: (reference ``numerical.py:20-25``).
DTYPE_RTOL: dict[torch.dtype, float] = {
    torch.float64: 1e-7,
    torch.float32: 1.3e-6,
    torch.float16: 1e-3,
    torch.bfloat16: 1.6e-2,
}

#: Absolute floor of every budget so that near-zero outputs are not compared to 0.
DEFAULT_ATOL = 1e-5

#: rtol used for a dtype missing from ``DTYPE_RTOL`` (reference ``numerical.py:113``).
FALLBACK_RTOL = 1e-3


def max_abs_error(a: torch.Tensor, b: torch.Tensor) -> float:
    """Largest elementwise ``|a - b|``, evaluated in fp32 (0.0 for empty tensors)."""
    if a.numel() == 0 and b.numel() == 0:
        return 0.0
    return (a.float() - b.float()).abs().max().item()


def max_abs_error_any(a: Any, b: Any) -> float:
    """``max_abs_error`` over a tensor or a (nested) sequence of tensors."""
    if isinstance(a, torch.Tensor) and isinstance(b, torch.Tensor):
        return max_abs_error(a, b)
    if isinstance(a, Sequence) and isinstance(b, Sequence):
        if len(a) != len(b):
            raise ValueError(f"Output arity mismatch: {len(a)} vs {len(b)}")
        return max((max_abs_error_any(x, y) for x, y in zip(a, b)), default=0.0)
    raise TypeError(f"Cannot compare outputs of types {type(a)!r} and {type(b)!r}")


def max_rel_error(a: torch.Tensor, b: torch.Tensor, eps: float = 1e-8) -> float:
    """Largest elementwise ``|a - b| / max(|a|, eps)``."""
    denom = a.float().abs().clamp_min(eps)
    return ((a.float() - b.float()).abs() / denom).max().item()


def assert_close(
    a: torch.Tensor, b: torch.Tensor, *, atol: float = 1e-2, rtol: float = 1e-2
) -> None:
    """Thin alias of ``torch.testing.assert_close`` with the reference's defaults."""
    torch.testing.assert_close(a, b, atol=atol, rtol=rtol)


def _max_magnitude(reference: Any) -> tuple[float, torch.dtype]:
    """``(max |reference|, dtype)``; for sequences the dtype of the first item."""
    if isinstance(reference, torch.Tensor):
        mag = reference.float().abs().max().item() if reference.numel() else 0.0
        return mag, reference.dtype
    if isinstance(reference, Sequence) and len(reference) > 0:
        parts = [_max_magnitude(item) for item in reference]
        return max(m for m, _ in parts), parts[0][1]
    raise TypeError(f"Cannot measure magnitude of {type(reference)!r}")


def ulp(dtype: torch.dtype, magnitude: float) -> float:
    """Spacing of representable ``dtype`` values in the binade of ``magnitude``.

    ``2**floor(log2 |m|) * eps(dtype)``, or the smallest normal when ``|m|`` is
    below it. An error under one ulp is a rounding difference, not a bug.
    """
    info = torch.finfo(dtype)
    magnitude = abs(magnitude)
    if magnitude < info.tiny:
        return info.tiny
    exponent = math.frexp(magnitude)[1] - 1  # floor(log2 m), exact for any float
    return math.ldexp(info.eps, exponent)


def error_budget(
    reference: Any,
    *,
    rtol: float | None = None,
    atol: float = DEFAULT_ATOL,
    tol_scale: float = 1.0,
) -> float:
    """Largest absolute disagreement two correct implementations may show."""
    magnitude, dtype = _max_magnitude(reference)
    if rtol is None:
        rtol = DTYPE_RTOL.get(dtype, FALLBACK_RTOL)
    return tol_scale * (atol + rtol * magnitude)


def error_in_ulps(reference: Any, candidate: Any) -> float:
    """Max absolute error in units of the output dtype's spacing at ``max|ref|``."""
    magnitude, dtype = _max_magnitude(reference)
    return max_abs_error_any(reference, candidate) / ulp(dtype, magnitude)


def ulp_report(reference: Any, candidate: Any, *, kernel: str = "candidate") -> dict[str, Any]:
    """Everything the gate decides on for one candidate, as a JSON-able dict."""
    magnitude, dtype = _max_magnitude(reference)
    err = max_abs_error_any(reference, candidate)
    budget = error_budget(reference)
    return {
        "kernel": kernel,
        "dtype": str(dtype).replace("torch.", ""),
        "max_abs_ref": magnitude,
        "max_error": err,
        "error_budget": budget,
        "ulp": ulp(dtype, magnitude),
        "err_ulps": err / ulp(dtype, magnitude),
        "budget_ulps": budget / ulp(dtype, magnitude),
        "passed": err <= budget,
    }
