"""Registration of every candidate into the process-wide registry.

Mirrors ``ako/ops/_registry.py:21-123`` with the Triton block replaced by the
HIP kernels of this package:

==========================  =================  ========  ===============
kernel                      backend            priority  registered when
==========================  =================  ========  ===============
``*_ref`` (unfused torch)   ``pytorch``        10        always
``rmsnorm_torch_native``    ``torch_native``   7         ``F.rms_norm`` exists
``*_compiled``              ``torch_compile``  7         ``AKO_ENABLE_COMPILE=1``
``*_hip``                   ``hip``            5         unless ``AKO_HIP_DISABLE=1``
==========================  =================  ========  ===============

One operation is added to the reference's four: ``rope_qk`` (query and key
rotated by the same tables). Its reference is ``rope_qk_ref`` (two
``rope_ref`` calls, ``ako/ops/rope_ref.py:110-118``); its HIP candidate
rotates both tensors in one launch.

The reference kernel has the highest priority, so with autotuning off (or on
a CPU tensor) the safe unfused path is the default and the HIP kernels have
to win a gated benchmark to be used. If the HIP library cannot be loaded
while a GPU is present, registration raises instead of silently racing only
the PyTorch baselines; on a machine without a GPU the HIP candidates are
simply left out (they could only raise there).
"""

from __future__ import annotations

import logging
import os

import torch

from ako_amd.dispatcher.registry import KernelEntry, KernelRegistry, get_registry

logger = logging.getLogger(__name__)

_PYTORCH_PRIORITY = 10
_BASELINE_PRIORITY = 7
_HIP_PRIORITY = 5

_registered = False


def hip_disabled() -> bool:
    return os.environ.get("AKO_HIP_DISABLE", "").strip().lower() in {"1", "true", "yes", "on"}


def _hip_entries() -> list[tuple[str, str, object]]:
    from ako_amd import _native

    try:
        _native.load()
    except _native.HipLibraryError:
        if torch.cuda.is_available():
            raise
        logger.info("HIP kernel library not loadable and no GPU present; HIP candidates skipped")
        return []
    from ako_amd.ops.rmsnorm_hip import rmsnorm_hip, rmsnorm_residual_hip
    from ako_amd.ops.rope_hip import rope_hip, rope_qk_hip
    from ako_amd.ops.swiglu_hip import swiglu_hip

    return [
        ("rmsnorm", "rmsnorm_hip", rmsnorm_hip),
        ("rmsnorm_residual", "rmsnorm_residual_hip", rmsnorm_residual_hip),
        ("rope", "rope_hip", rope_hip),
        ("rope_qk", "rope_qk_hip", rope_qk_hip),
        ("swiglu", "swiglu_hip", swiglu_hip),
    ]


def register_all(registry: KernelRegistry | None = None, *, force: bool = False) -> KernelRegistry:
    """Register references, baselines and HIP kernels for every operation (idempotent)."""
    global _registered
    target = registry if registry is not None else get_registry()
    if registry is None and _registered and not force:
        return target

    from ako_amd.ops.rmsnorm_ref import rmsnorm_ref, rmsnorm_residual_ref
    from ako_amd.ops.rmsnorm_torch import (
        is_compile_enabled,
        is_native_available,
        rmsnorm_compiled,
        rmsnorm_residual_compiled,
        rmsnorm_torch_native,
        rope_compiled,
        swiglu_compiled,
    )
    from ako_amd.ops.rope_ref import rope_qk_ref, rope_ref
    from ako_amd.ops.swiglu_ref import swiglu_ref

    entries: list[KernelEntry] = [
        KernelEntry(op, name, fn, backend="pytorch", priority=_PYTORCH_PRIORITY)
        for op, name, fn in (
            ("rmsnorm", "rmsnorm_ref", rmsnorm_ref),
            ("rmsnorm_residual", "rmsnorm_residual_ref", rmsnorm_residual_ref),
            ("rope", "rope_ref", rope_ref),
            ("rope_qk", "rope_qk_ref", rope_qk_ref),
            ("swiglu", "swiglu_ref", swiglu_ref),
        )
    ]
    if is_native_available():
        entries.append(
            KernelEntry("rmsnorm", "rmsnorm_torch_native", rmsnorm_torch_native,
                        backend="torch_native", priority=_BASELINE_PRIORITY)
        )
    if is_compile_enabled():
        entries += [
            KernelEntry(op, name, fn, backend="torch_compile", priority=_BASELINE_PRIORITY)
            for op, name, fn in (
                ("rmsnorm", "rmsnorm_compiled", rmsnorm_compiled),
                ("rmsnorm_residual", "rmsnorm_residual_compiled", rmsnorm_residual_compiled),
                ("rope", "rope_compiled", rope_compiled),
                ("swiglu", "swiglu_compiled", swiglu_compiled),
            )
        ]
    if not hip_disabled():
        entries += [
            KernelEntry(op, name, fn, backend="hip", priority=_HIP_PRIORITY)
            for op, name, fn in _hip_entries()
        ]
    for entry in entries:
        target.register(entry)

    if registry is None:
        _registered = True
        from ako_amd.dispatcher.selector import get_selector

        get_selector().clear_memo()  # a re-registration must not keep stale picks
    return target


def reset_registration() -> None:
    """Allow :func:`register_all` to run again (tests)."""
    global _registered
    _registered = False
