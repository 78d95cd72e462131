"""The amdgpu driver's sysfs view of one GPU, matched to a torch device index.

torch numbers the GPUs it sees (after ``HIP_VISIBLE_DEVICES`` remapping), the
DRM subsystem numbers cards (``/sys/class/drm/cardN``) and the KFD numbers
compute nodes (``/sys/class/kfd/kfd/topology/nodes/N``, each with a
``gpu_id``). None of these orders has to agree with another, so a device is
matched by its PCI address, which all three report:

- torch: ``pci_domain_id``, ``pci_bus_id``, ``pci_device_id`` of the device
  properties;
- DRM: ``PCI_SLOT_NAME=DDDD:BB:DD.F`` in ``cardN/device/uevent``;
- KFD: ``domain`` and ``location_id`` (``bus << 8 | device << 3 | function``)
  in ``nodes/N/properties``.

Only when torch gives no PCI address (no GPU build, or an older torch) does a
device index fall back to its position among the cards, sorted by card
number (``card2`` before ``card10``). Every function returns ``None`` (or an
empty list) when the files it needs are missing: a sandbox that hides sysfs
still measures, it only records less.
"""

from __future__ import annotations

import re
from pathlib import Path

DRM = Path("/sys/class/drm")
KFD_TOPOLOGY = Path("/sys/class/kfd/kfd/topology/nodes")
KFD_PROCS = Path("/sys/class/kfd/kfd/proc")


def _read(path: Path) -> str | None:
    try:
        return path.read_text().strip()
    except OSError:
        return None


def card_device_dirs(drm: Path = DRM, marker: str | None = None) -> list[Path]:
    """``cardN/device`` directories in card-number order (``card2`` before
    ``card10``), only those with a file named ``marker`` when one is given."""
    cards = [p for p in drm.glob("card[0-9]*") if re.fullmatch(r"card\d+", p.name)]
    cards.sort(key=lambda p: int(p.name[4:]))
    devs = [c / "device" for c in cards]
    return [d for d in devs if marker is None or (d / marker).exists()]


def pci_slot_name(domain: int, bus: int, device: int, function: int = 0) -> str:
    """The kernel's PCI address format, ``DDDD:BB:DD.F`` in lower-case hex."""
    return f"{domain:04x}:{bus:02x}:{device:02x}.{function:x}"


def torch_pci_slot(index: int) -> str | None:
    """PCI address of torch's GPU ``index``, or None when torch has no GPU or
    no PCI fields."""
    try:
        import torch

        if not torch.cuda.is_available():
            return None
        props = torch.cuda.get_device_properties(index)
        return pci_slot_name(int(props.pci_domain_id), int(props.pci_bus_id), int(props.pci_device_id))
    except (AttributeError, RuntimeError, AssertionError, ValueError, TypeError):
        return None


def _uevent_slot(dev: Path) -> str | None:
    for line in (_read(dev / "uevent") or "").splitlines():
        if line.startswith("PCI_SLOT_NAME="):
            return line.split("=", 1)[1].strip().lower()
    return None


def device_dir(index: int, *, drm: Path = DRM, marker: str | None = None,
               slot: str | None = None) -> Path | None:
    """The ``cardN/device`` directory of torch's GPU ``index``: the card whose
    PCI address is ``slot`` (by default torch's own for ``index``); without an
    address, the ``index``-th card in card-number order."""
    devs = card_device_dirs(drm, marker)
    slot = slot if slot is not None else torch_pci_slot(index)
    if slot is not None:
        for dev in devs:
            if _uevent_slot(dev) == slot.lower():
                return dev
        return None
    return devs[index] if 0 <= index < len(devs) else None


def peak_sclk_khz(dev: Path) -> int | None:
    """The highest engine-clock level in ``pp_dpm_sclk`` (lines like
    ``1: 2400Mhz *``), in kHz: the same figure as HIP's ``clockRate``."""
    levels = [int(m.group(1)) for m in re.finditer(r"(\d+)\s*Mhz", _read(dev / "pp_dpm_sclk") or "", re.IGNORECASE)]
    return max(levels) * 1000 if levels else None


def kfd_gpu_id(slot: str, topology: Path = KFD_TOPOLOGY) -> int | None:
    """The KFD ``gpu_id`` of the node at PCI address ``slot`` (CPU nodes have
    gpu_id 0 and are skipped)."""
    m = re.fullmatch(r"([0-9a-f]{4}):([0-9a-f]{2}):([0-9a-f]{2})\.([0-7])", slot.lower())
    if m is None:
        return None
    domain, bus, dev, fn = (int(g, 16) for g in m.groups())
    location = (bus << 8) | (dev << 3) | fn
    try:
        nodes = list(topology.iterdir())
    except OSError:
        return None
    for node in nodes:
        gpu_id = _read(node / "gpu_id")
        if not gpu_id or gpu_id == "0":
            continue
        props = {}
        for line in (_read(node / "properties") or "").splitlines():
            parts = line.split()
            if len(parts) == 2 and parts[1].lstrip("-").isdigit():
                props[parts[0]] = int(parts[1])
        if props.get("location_id") == location and props.get("domain", 0) == domain:
            return int(gpu_id)
    return None


def kfd_processes(gpu_id: int | None = None, kfd_proc: Path = KFD_PROCS) -> list[int] | None:
    """PIDs with a KFD compute context, or None when the KFD is not visible.

    With ``gpu_id``, only processes with a per-device entry for that GPU: a
    process directory lists entries named ``<what>_<gpu_id>`` (``vram_``,
    ``sdma_``, ``stats_``) for each GPU it has opened, and a HIP process
    typically opens every GPU it can see, so this rules out processes
    confined to other GPUs (``HIP_VISIBLE_DEVICES``). A directory with no
    per-device entries at all is counted, since it cannot be ruled out."""
    try:
        entries = [p for p in kfd_proc.iterdir() if p.name.isdigit()]
    except OSError:
        return None
    pids = []
    for proc in entries:
        if gpu_id is not None:
            try:
                names = [p.name for p in proc.iterdir()]
            except OSError:
                names = []
            per_gpu = [n for n in names if re.fullmatch(r"[a-z]+_\d+", n)]
            if per_gpu and not any(n.endswith(f"_{gpu_id}") for n in per_gpu):
                continue
        pids.append(int(proc.name))
    return sorted(pids)
