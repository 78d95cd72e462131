"""Numerical validation: the dtype-aware gate and ulp reports."""

from ako_amd.validation.numerical import (
    DEFAULT_ATOL,
    DTYPE_RTOL,
    assert_close,
    error_budget,
    error_in_ulps,
    max_abs_error,
    max_abs_error_any,
    max_rel_error,
    ulp,
    ulp_report,
)

__all__ = [
    "DEFAULT_ATOL",
    "DTYPE_RTOL",
    "assert_close",
    "error_budget",
    "error_in_ulps",
    "max_abs_error",
    "max_abs_error_any",
    "max_rel_error",
    "ulp",
    "ulp_report",
]
