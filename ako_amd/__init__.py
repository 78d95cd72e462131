"""AKO's candidate kernels, MI355X-native.

Public operations keep the signatures of Farx1/AKO's ``ako`` package
(``ako/__init__.py:5-17``); kernel choice goes through the same gated,
benchmark-driven selector, and the gfx950 HIP kernels race the PyTorch
baselines as ``backend="hip"`` candidates. ``rope_qk_cache`` (RoPE of q and k
plus the KV-cache append in one launch) is an addition of this package; it
writes the caches in place, so it is called directly rather than selected.
"""

__version__ = "0.1.0"

from ako_amd.ops.rmsnorm import rmsnorm, rmsnorm_residual
from ako_amd.ops.rope import build_rope_tables, rope, rope_qk, rope_qk_cache
from ako_amd.ops.swiglu import swiglu

__all__ = [
    "__version__",
    "build_rope_tables",
    "rmsnorm",
    "rmsnorm_residual",
    "rope",
    "rope_qk",
    "rope_qk_cache",
    "swiglu",
]
