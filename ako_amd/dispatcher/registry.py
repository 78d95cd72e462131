"""Kernel registry: the plugin API every candidate sits behind.

Same contract as ``ako/dispatcher/registry.py:13-60``: a ``KernelEntry`` names
an operation, a kernel, a callable, a backend string and a priority.
Registering a name that already exists for the operation replaces it, and each
operation's list is kept sorted by descending priority, so ``default(op)`` is
the highest-priority kernel (the PyTorch reference, priority 10, in practice).

``backend="pytorch"`` is reserved for the numerical reference of an operation;
``torch_native`` and ``torch_compile`` are the other baselines; the HIP kernels
of this package register as ``backend="hip"``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

KernelFn = Callable[..., torch.Tensor]


@dataclass(frozen=True)
class KernelEntry:
    """One registered implementation of one operation."""

    op_name: str
    kernel_name: str
    fn: KernelFn
    backend: str
    priority: int = 0


class KernelRegistry:
    """Per-operation lists of kernels, highest priority first."""

    def __init__(self) -> None:
        self._by_op: dict[str, list[KernelEntry]] = {}

    def register(self, entry: KernelEntry) -> None:
        """Insert ``entry``; an entry of the same operation and name is replaced."""
        kept = [e for e in self._by_op.get(entry.op_name, []) if e.kernel_name != entry.kernel_name]
        kept.append(entry)
        # sorted() is stable: equal priorities keep their registration order.
        self._by_op[entry.op_name] = sorted(kept, key=lambda e: -e.priority)

    def unregister(self, op_name: str, kernel_name: str) -> bool:
        """Drop one kernel; returns whether it was present."""
        entries = self._by_op.get(op_name, [])
        kept = [e for e in entries if e.kernel_name != kernel_name]
        self._by_op[op_name] = kept
        return len(kept) != len(entries)

    def list_ops(self) -> list[str]:
        return sorted(op for op, entries in self._by_op.items() if entries)

    def list_kernels(self, op_name: str) -> list[KernelEntry]:
        return list(self._by_op.get(op_name, ()))

    def get(self, op_name: str, kernel_name: str) -> KernelEntry | None:
        return next((e for e in self._by_op.get(op_name, ()) if e.kernel_name == kernel_name), None)

    def default(self, op_name: str) -> KernelEntry | None:
        entries = self._by_op.get(op_name)
        return entries[0] if entries else None


_GLOBAL_REGISTRY = KernelRegistry()


def get_registry() -> KernelRegistry:
    """The process-wide registry used by the public ``ako_amd`` operations."""
    return _GLOBAL_REGISTRY
