"""Device introspection for the cache key and the reports, ROCm-native.

Replaces ``ako/dispatcher/hardware.py:22-193`` of the reference, which read
CUDA attributes through ``ctypes.CDLL("libcudart.so")`` and the driver through
``nvidia-smi``. Here everything comes from the HIP runtime that PyTorch-ROCm
already initialised: ``hipGetDeviceProperties`` and ``hipDriverGetVersion``
through the library's ``ako_device_identity``, or torch's property object when
the library is not loaded. No subprocess runs on the dispatch path. The
``DeviceInfo`` fields and the ``cache_key`` format
(``"<name with _ for spaces>_<index>"``) are the reference's, so cache files
stay keyed the same way.

The reference keys selections by the product name (``hardware.py:60-63``). On
ROCm the name HIP reports can be the generic "AMD Radeon Graphics" for every
part, so ``device_name`` here is that name followed by the fields that tell
parts apart: the ISA, the compute-unit count, the peak engine clock and the
HBM size (``"AMD Radeon Graphics gfx950 256CU 2400MHz 288GB"``). An MI300X
(gfx942, 304 CUs) and an MI355X (gfx950, 256 CUs, 2400 MHz) never share a key,
nor do an MI350X and an MI355X (the same ISA and CU count, 2200 against
2400 MHz). Some boxes report an empty name instead of the generic one for the
same part; ``part_label`` maps both to "AMD Radeon Graphics", so the key does
not change from box to box.

The clock comes from HIP's ``clockRate`` when the library is loaded, else from
the highest level of the card's ``pp_dpm_sclk`` (the card matched by PCI
address, ``amdgpu_sysfs``); the two agree (2400 MHz on MI355X). An identity
still missing its clock is not memoised, so a process that asks before the
library loads does not keep a key that other processes never use.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from functools import lru_cache
from pathlib import Path

import torch

from ako_amd.dispatcher import amdgpu_sysfs


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
    #: The name exactly as HIP reports it (``device_name`` adds the part fields).
    marketing_name: str | None = None
    #: Peak engine clock in MHz (``hipDeviceProp_t.clockRate``).
    clock_mhz: int | None = None

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
def _amdgpu_module_version() -> str | None:
    """The amdgpu kernel-module version from sysfs, where the module has one
    (a DKMS build does; the in-tree module of many kernels does not)."""
    try:
        text = Path("/sys/module/amdgpu/version").read_text().strip()
    except OSError:
        return None
    return text or None


def driver_label(module_version: str | None, hip_driver: int | None) -> str | None:
    """``"amdgpu <version>"`` when the module reports one, else the HIP driver
    version (``hipDriverGetVersion``, which every ROCm install answers)."""
    if module_version:
        return f"amdgpu {module_version}"
    if hip_driver is not None and hip_driver > 0:
        return f"hip {hip_driver}"
    return None


GENERIC_AMD_NAME = "AMD Radeon Graphics"
_GENERIC_AMD_NAMES = {"", "amd radeon graphics", "amd gpu"}


def part_label(name: str, arch: str | None, cus: int | None, clock_khz: int | None,
               mem_bytes: int | None) -> str:
    """HIP's device name followed by the fields that tell parts apart:
    ``"<name> <isa> <cus>CU <MHz>MHz <GiB>GB"``; missing fields are left out.

    Some boxes report the generic "AMD Radeon Graphics", others an empty name,
    for the same part; both carry no information, so both become
    ``GENERIC_AMD_NAME`` and one part keeps one cache key across boxes."""
    base = name.strip()
    parts = [GENERIC_AMD_NAME if base.lower() in _GENERIC_AMD_NAMES else base]
    if arch:
        parts.append(arch.split(":")[0])
    if cus:
        parts.append(f"{int(cus)}CU")
    if clock_khz and clock_khz > 0:
        parts.append(f"{int(round(clock_khz / 1000))}MHz")
    if mem_bytes and mem_bytes > 0:
        parts.append(f"{int(round(mem_bytes / 1024**3))}GB")
    return " ".join(parts)


def _hip_identity(index: int) -> dict[str, str] | None:
    """``ako_device_identity`` fields, or None when the library is not usable."""
    try:
        from ako_amd import _native

        return _native.device_identity(index)
    except Exception:  # noqa: BLE001 - a missing library falls back to torch's props
        return None


def _int_or_none(text: str | None) -> int | None:
    try:
        return int(text) if text not in (None, "") else None
    except ValueError:
        return None


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


_INFO_CACHE: dict[tuple[str, int | None], DeviceInfo] = {}


def clear_device_cache() -> None:
    """Forget memoised probes (tests)."""
    _INFO_CACHE.clear()
    _compute_backend.cache_clear()
    _amdgpu_module_version.cache_clear()


def sysfs_clock_khz(index: int) -> int | None:
    """Peak engine clock of torch's GPU ``index`` from the card's
    ``pp_dpm_sclk``, or None when sysfs does not show it."""
    dev = amdgpu_sysfs.device_dir(index, marker="pp_dpm_sclk")
    return amdgpu_sysfs.peak_sclk_khz(dev) if dev is not None else None


def _device_info(device_type: str, device_index: int | None) -> DeviceInfo:
    key = (device_type, device_index)
    cached = _INFO_CACHE.get(key)
    if cached is not None:
        return cached
    info = _probe_device(device_type, device_index)
    # A ROCm identity without its clock (no library, no sysfs) is answered
    # but not kept: a later call, once either source is there, gets the key
    # that every other process uses.
    if info.compute_backend != "rocm" or info.clock_mhz is not None:
        _INFO_CACHE[key] = info
    return info


def _probe_device(device_type: str, device_index: int | None) -> DeviceInfo:
    backend = _compute_backend()
    if device_type == "cuda" and torch.cuda.is_available():
        index = device_index or 0
        props = torch.cuda.get_device_properties(index)
        ident = _hip_identity(index) if backend == "rocm" else None
        ident = ident or {}
        arch = ident.get("arch") or getattr(props, "gcnArchName", None)
        cus = _int_or_none(ident.get("cus")) or getattr(props, "multi_processor_count", None)
        clock_khz = _int_or_none(ident.get("clock_khz"))
        if clock_khz is None and backend == "rocm":
            clock_khz = sysfs_clock_khz(index)
        mem_bytes = _int_or_none(ident.get("mem_bytes")) or props.total_memory
        raw_name = ident.get("name") or props.name
        name = part_label(raw_name, arch, cus, clock_khz, mem_bytes) if backend == "rocm" else props.name
        driver = (driver_label(_amdgpu_module_version(), _int_or_none(ident.get("hip_driver")))
                  if backend == "rocm" else None)
        return DeviceInfo(
            device_type="cuda",
            device_name=name,
            device_index=index,
            cuda_capability=(props.major, props.minor),
            total_memory_gb=round(props.total_memory / 1024**3, 2),
            driver_version=driver,
            gpu_vendor="amd" if backend == "rocm" else "nvidia",
            compute_backend=backend,
            sm_count=getattr(props, "multi_processor_count", None),
            smem_per_block=(
                getattr(props, "shared_memory_per_block_optin", None)
                or getattr(props, "shared_memory_per_block", None)
            ),
            l2_bytes=getattr(props, "L2_cache_size", None),
            regs_per_sm=getattr(props, "regs_per_multiprocessor", None),
            gcn_arch=arch,
            hip_runtime=getattr(torch.version, "hip", None),
            marketing_name=raw_name,
            clock_mhz=int(round(clock_khz / 1000)) if clock_khz else None,
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
