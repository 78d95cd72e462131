"""Adaptive kernel dispatch: device introspection, registry, selection, cache."""

from ako_amd.dispatcher.cache import KernelCache
from ako_amd.dispatcher.hardware import get_device_info
from ako_amd.dispatcher.registry import KernelEntry, KernelRegistry, get_registry
from ako_amd.dispatcher.selector import KernelSelector, get_selector, reset_selector

__all__ = [
    "KernelCache",
    "KernelEntry",
    "KernelRegistry",
    "KernelSelector",
    "get_device_info",
    "get_registry",
    "get_selector",
    "reset_selector",
]
