"""GPU state next to a measurement: clock, temperature, power.

The reference samples these through ``nvidia-smi`` (``ako/benchmark/env.py:80-119``).
On ROCm the amdgpu driver exposes them in sysfs, which needs no subprocess:
``pp_dpm_sclk`` (the active shader clock is the line marked ``*``) and the
hwmon ``temp*_input`` (millidegrees) / ``power1_average`` or ``power1_input``
(microwatts). Every field is ``None`` when the file is missing, because a
measurement without an environment sample is still a measurement.
"""

from __future__ import annotations

import os
import re
from pathlib import Path
from typing import Any

_DRM = Path("/sys/class/drm")


def _gpu_device_dirs() -> list[Path]:
    cards = sorted(p for p in _DRM.glob("card[0-9]*") if re.fullmatch(r"card\d+", p.name))
    return [c / "device" for c in cards if (c / "device" / "pp_dpm_sclk").exists()]


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


def sample_env(index: int = 0) -> dict[str, Any]:
    """Clock (MHz), temperature (C) and power (W) of GPU ``index``, or ``None``s."""
    devices = _gpu_device_dirs()
    if index >= len(devices):
        return {"sm_clock_mhz": None, "temp_c": None, "power_w": None, "throttle_reasons": None}
    dev = devices[index]
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
