"""GPU state next to a measurement: clock, temperature, power, idleness.

The reference samples these through ``nvidia-smi`` (``ako/benchmark/env.py:80-119``).
On ROCm the amdgpu driver exposes them in sysfs, which needs no subprocess:
``pp_dpm_sclk`` (the active shader clock is the line marked ``*``) and the
hwmon ``temp*_input`` (millidegrees) / ``power1_average`` or ``power1_input``
(microwatts). Every field is ``None`` when the file is missing, because a
measurement without an environment sample is still a measurement.

``preflight`` is the reference's busy-GPU check (``env.py:95-119``): other
processes computing on the card, or a card already busy, make every latency
measured after it meaningless. On ROCm the compute processes are the entries
of the KFD's ``/sys/class/kfd/kfd/proc`` (one directory per process with a GPU
context) and the load is the card's ``gpu_busy_percent``.
"""

from __future__ import annotations

import os
import re
from pathlib import Path
from typing import Any

from ako_amd.dispatcher import amdgpu_sysfs

_DRM = amdgpu_sysfs.DRM


def _read(path: Path) -> str | None:
    try:
        return path.read_text().strip()
    except OSError:
        return None


def _active_sclk_mhz(dev: Path) -> float | None:
    text = _read(dev / "pp_dpm_sclk")
    for line in (text or "").splitlines():
        if line.rstrip().endswith("*"):
            match = re.search(r"(\d+)\s*Mhz", line, re.IGNORECASE)
            if match:
                return float(match.group(1))
    return None


def _hwmon_value(dev: Path, names: tuple[str, ...], scale: float) -> float | None:
    for hwmon in sorted((dev / "hwmon").glob("hwmon*")):
        for name in names:
            raw = _read(hwmon / name)
            if raw is not None:
                try:
                    return float(raw) / scale
                except ValueError:
                    continue
    return None


def sample_env(index: int = 0, *, drm: Path = _DRM, slot: str | None = None) -> dict[str, Any]:
    """Clock (MHz), temperature (C) and power (W) of torch's GPU ``index`` (the
    card at its PCI address, ``amdgpu_sysfs.device_dir``), or ``None``s."""
    dev = amdgpu_sysfs.device_dir(index, drm=drm, marker="pp_dpm_sclk", slot=slot)
    if dev is None:
        return {"sm_clock_mhz": None, "temp_c": None, "power_w": None, "throttle_reasons": None}
    return {
        "sm_clock_mhz": _active_sclk_mhz(dev),
        "temp_c": _hwmon_value(dev, ("temp1_input", "temp2_input"), 1e3),
        "power_w": _hwmon_value(dev, ("power1_average", "power1_input"), 1e6),
        "throttle_reasons": None,
    }


def host_cpu() -> dict[str, Any]:
    """Host CPU facts for the CPU-baseline columns."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": affinity}


_KFD_PROCS = amdgpu_sysfs.KFD_PROCS
_KFD_TOPOLOGY = amdgpu_sysfs.KFD_TOPOLOGY
#: Utilisation at or above which the card is taken to be busy (the reference's 3%).
BUSY_PERCENT = 3.0


def _busy_percent(dev: Path) -> float | None:
    raw = _read(dev / "gpu_busy_percent")
    try:
        return float(raw) if raw is not None else None
    except ValueError:
        return None


def gpu_processes(kfd_proc: Path = _KFD_PROCS, gpu_id: int | None = None) -> list[int] | None:
    """PIDs with a GPU compute context (on the KFD node ``gpu_id`` when
    given, else on any GPU), or None when the KFD is not visible."""
    return amdgpu_sysfs.kfd_processes(gpu_id, kfd_proc)


def preflight(index: int = 0, *, strict: bool = True, kfd_proc: Path = _KFD_PROCS,
              drm: Path | None = None, topology: Path = _KFD_TOPOLOGY,
              slot: str | None = None) -> dict[str, Any]:
    """Check that torch's GPU ``index`` is idle before measuring.

    The card and the KFD node are the ones at the device's PCI address
    (``slot``, by default torch's); processes are counted on that GPU only
    when its KFD node is found, else on any GPU. Returns
    ``{"checked", "compute_apps", "utilization_gpu"}``; ``checked`` is False
    when neither source is readable (a sandbox that hides sysfs). With
    ``strict`` a busy card raises ``RuntimeError`` (the reference's
    behaviour); otherwise the state is returned with ``"busy": True`` for the
    caller to record next to its numbers.
    """
    slot = slot if slot is not None else amdgpu_sysfs.torch_pci_slot(index)
    dev = amdgpu_sysfs.device_dir(index, drm=drm if drm is not None else _DRM, marker="gpu_busy_percent",
                                  slot=slot)
    used = _busy_percent(dev) if dev is not None else None
    gpu_id = amdgpu_sysfs.kfd_gpu_id(slot, topology) if slot is not None else None
    pids = gpu_processes(kfd_proc, gpu_id)
    mine = os.getpid()
    foreign = [p for p in (pids or []) if p != mine]
    state: dict[str, Any] = {"checked": used is not None or pids is not None,
                             "compute_apps": foreign, "utilization_gpu": used}
    problems = []
    if foreign:
        problems.append(f"other processes hold GPU contexts: {foreign}")
    if used is not None and used >= BUSY_PERCENT:
        problems.append(f"gpu_busy_percent = {used:.0f}% (want < {BUSY_PERCENT:.0f}%)")
    state["busy"] = bool(problems)
    if problems and strict:
        raise RuntimeError("GPU is not idle: " + "; ".join(problems))
    return state


def report() -> dict[str, Any]:
    """What ``python -m ako_amd.benchmark.env`` prints: the runtime, the device,
    whether the HIP library and its binding load, and whether the GPU is idle
    (the reference's ``scripts/check_environment.py``, ROCm-side)."""
    import sys

    import torch

    from ako_amd import _native
    from ako_amd.dispatcher.hardware import get_device_info

    info = get_device_info()
    out: dict[str, Any] = {
        "python": sys.version.split()[0],
        "torch": torch.__version__,
        "hip_runtime": getattr(torch.version, "hip", None),
        "gpu_available": torch.cuda.is_available(),
        "compute_backend": info.compute_backend,
        "device": info.device_name,
        "cache_key": info.cache_key,
        "driver": info.driver_version,
        "host": host_cpu(),
    }
    try:
        lib = _native.load()
        out["hip_library"] = lib.ako_build_info().decode()
    except _native.HipLibraryError as exc:
        out["hip_library"] = f"not loadable: {exc}"
    try:
        out["torch_binding"] = _native.torch_binding() is not None
    except _native.HipLibraryError:
        out["torch_binding"] = False
    if torch.cuda.is_available():
        out["preflight"] = preflight(torch.cuda.current_device(), strict=False)
        out["gpu_state"] = sample_env(torch.cuda.current_device())
    return out


def main(argv: list[str] | None = None) -> int:
    import json

    state = report()
    width = max(len(k) for k in state)
    for key, value in state.items():
        shown = json.dumps(value) if isinstance(value, (dict, list)) else str(value)
        print(f"{key:<{width}}  {shown}")
    if not state["gpu_available"]:
        print("\nCPU only: the oracle, the gate, the selector and the ABI checks run here "
              "(pytest -m 'not gpu'); the HIP kernels need an MI355X (gfx950).")
    elif str(state["hip_library"]).startswith("not loadable"):
        print("\nThe GPU is visible but the kernel library is not built: "
              "python -c 'import __graft_entry__ as g; g.build()'")
        return 1
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
