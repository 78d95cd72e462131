"""LLM building-block operations: references, baselines, HIP candidates, dispatch."""

from ako_amd.ops.rmsnorm import rmsnorm, rmsnorm_residual
from ako_amd.ops.rope import build_rope_tables, rope, rope_qk
from ako_amd.ops.swiglu import swiglu

__all__ = ["build_rope_tables", "rmsnorm", "rmsnorm_residual", "rope", "rope_qk", "swiglu"]
