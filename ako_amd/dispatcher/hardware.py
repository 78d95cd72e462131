"""Device introspection for the cache key and the reports, ROCm-native.

Replaces ``ako/dispatcher/hardware.py:22-193`` of the reference, which read
CUDA attributes through ``ctypes.CDLL("libcudart.so")`` and the driver through
``nvidia-smi``. Here everything comes from the HIP runtime that PyTorch-ROCm
already initialised (``torch.cuda.get_device_properties`` is a thin wrapper of
``hipGetDeviceProperties``) plus the amdgpu kernel module's version file, so
no subprocess runs on the dispatch path. The ``DeviceInfo`` fields and the
``cache_key`` format (``"<name with _ for spaces>_<index>"``) are the
reference's, so cache files stay keyed the same way.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from functools import lru_cache
from pathlib import Path

import torch


@dataclass(frozen=True)
class DeviceInfo:
    """Snapshot of one compute device."""

    device_type: str
    device_name: str
    device_index: int
    cuda_capability: tuple[int, int] | None
    total_memory_gb: float | None
    driver_version: str | None
    gpu_vendor: str | None = None
    compute_backend: str = "cpu"
    #: Compute units (the reference calls them SMs).
    sm_count: int | None = None
    #: LDS bytes one workgroup may allocate.
    smem_per_block: int | None = None
    l2_bytes: int | None = None
    regs_per_sm: int | None = None
    #: ``gcnArchName`` with feature flags, e.g. ``gfx950:sramecc+:xnack-``.
    gcn_arch: str | None = None
    hip_runtime: str | None = None

    @property
    def cache_key(self) -> str:
        return f"{self.device_name.replace(' ', '_')}_{self.device_index}"

    @property
    def arch(self) -> str | None:
        """The bare ISA name (``gfx950``) without feature flags."""
        return self.gcn_arch.split(":")[0] if self.gcn_arch else None

    def to_dict(self) -> dict:
        return asdict(self)


@lru_cache(maxsize=1)
def _compute_backend() -> str:
    if torch.cuda.is_available():
        return "rocm" if getattr(torch.version, "hip", None) else "cuda"
    return "cpu"


@lru_cache(maxsize=1)
def _amdgpu_driver_version() -> str | None:
    """The amdgpu kernel-module version, read from sysfs (no subprocess)."""
    try:
        text = Path("/sys/module/amdgpu/version").read_text().strip()
    except OSError:
        return None
    return text or None


def get_device_info(device: torch.device | str | None = None) -> DeviceInfo:
    """Metadata for ``device`` (default: the current accelerator, else CPU); memoised."""
    if device is None:
        device = (
            torch.device("cuda", torch.cuda.current_device())
            if torch.cuda.is_available()
            else torch.device("cpu")
        )
    elif isinstance(device, str):
        device = torch.device(device)
    index = device.index
    if device.type == "cuda" and index is None and torch.cuda.is_available():
        index = torch.cuda.current_device()
    return _device_info(device.type, index)


def clear_device_cache() -> None:
    """Forget memoised probes (tests)."""
    _device_info.cache_clear()
    _compute_backend.cache_clear()
    _amdgpu_driver_version.cache_clear()


@lru_cache(maxsize=None)
def _device_info(device_type: str, device_index: int | None) -> DeviceInfo:
    backend = _compute_backend()
    if device_type == "cuda" and torch.cuda.is_available():
        props = torch.cuda.get_device_properties(device_index or 0)
        return DeviceInfo(
            device_type="cuda",
            device_name=props.name,
            device_index=device_index or 0,
            cuda_capability=(props.major, props.minor),
            total_memory_gb=round(props.total_memory / 1024**3, 2),
            driver_version=_amdgpu_driver_version() if backend == "rocm" else None,
            gpu_vendor="amd" if backend == "rocm" else "nvidia",
            compute_backend=backend,
            sm_count=getattr(props, "multi_processor_count", None),
            smem_per_block=(
                getattr(props, "shared_memory_per_block_optin", None)
                or getattr(props, "shared_memory_per_block", None)
            ),
            l2_bytes=getattr(props, "L2_cache_size", None),
            regs_per_sm=getattr(props, "regs_per_multiprocessor", None),
            gcn_arch=getattr(props, "gcnArchName", None),
            hip_runtime=getattr(torch.version, "hip", None),
        )
    return DeviceInfo(
        device_type=device_type,
        device_name="cpu",
        device_index=-1,
        cuda_capability=None,
        total_memory_gb=None,
        driver_version=None,
        gpu_vendor=None,
        compute_backend="cpu",
    )
