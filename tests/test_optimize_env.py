"""Offline workload selection (``ako_amd.benchmark.optimize``) and the busy-GPU
preflight (``ako_amd.benchmark.env.preflight``), on the CPU."""

from __future__ import annotations

import json
import os

import pytest
import torch

from ako_amd.benchmark import env
from ako_amd.benchmark import optimize


def _fake_sysfs(tmp_path, busy: str | None, pids: list[int] | None):
    drm = tmp_path / "drm"
    dev = drm / "card0" / "device"
    dev.mkdir(parents=True)
    if busy is not None:
        (dev / "gpu_busy_percent").write_text(busy + "\n")
    kfd = tmp_path / "kfd_proc"
    if pids is not None:
        kfd.mkdir()
        for pid in pids:
            (kfd / str(pid)).mkdir()
    return drm, kfd


def test_preflight_idle_card(tmp_path) -> None:
    drm, kfd = _fake_sysfs(tmp_path, "0", [os.getpid()])
    state = env.preflight(drm=drm, kfd_proc=kfd)
    assert state == {"checked": True, "compute_apps": [], "utilization_gpu": 0.0, "busy": False}


def test_preflight_refuses_a_busy_card(tmp_path) -> None:
    drm, kfd = _fake_sysfs(tmp_path, "57", [os.getpid(), 4242])
    with pytest.raises(RuntimeError, match="not idle.*4242.*57%"):
        env.preflight(drm=drm, kfd_proc=kfd)
    state = env.preflight(drm=drm, kfd_proc=kfd, strict=False)
    assert state["busy"] and state["compute_apps"] == [4242] and state["utilization_gpu"] == 57.0
    # Just under the threshold is idle.
    drm2, kfd2 = _fake_sysfs(tmp_path / "b", "2", [])
    assert env.preflight(drm=drm2, kfd_proc=kfd2)["busy"] is False


def test_preflight_without_sysfs_is_unchecked(tmp_path) -> None:
    state = env.preflight(drm=tmp_path / "none", kfd_proc=tmp_path / "none")
    assert state == {"checked": False, "compute_apps": [], "utilization_gpu": None, "busy": False}


def test_workload_tensors_follow_the_decoder_layer() -> None:
    w = optimize.Workload(batch_size=2, seq_len=3, hidden_dim=64, num_heads=4, num_kv_heads=2, head_dim=16,
                          ffn_dim=96, dtype=torch.float32)
    t = w.tensors(torch.device("cpu"))
    assert set(t) == {"rmsnorm", "rmsnorm_residual", "rope", "rope_qk", "swiglu"}
    assert t["rmsnorm"][0][0].shape == (2, 3, 64) and t["rmsnorm"][0][1].shape == (64,)
    q, k, cos, sin = t["rope_qk"][0]
    assert q.shape == (2, 3, 4, 16) and k.shape == (2, 3, 2, 16) and cos.shape == (3, 8)
    assert t["rope"][1] == {"style": "neox"} and t["swiglu"][0][0].shape == (2, 3, 96)
    # Seeded: the same workload gives the same inputs.
    assert torch.equal(t["rmsnorm"][0][0], w.tensors(torch.device("cpu"))["rmsnorm"][0][0])
    phases = optimize.config5_phases()
    assert phases["prefill"].seq_len == 512 and phases["decode"].seq_len == 1
    assert phases["decode"].hidden_dim == 4096 and phases["decode"].ffn_dim == 11008


def test_optimize_writes_the_selected_config(tmp_path) -> None:
    """On the CPU the selector returns its default (only the baselines run
    there); the document still has the reference's layout, one operation per
    op, and the decisions are in the cache."""
    out = tmp_path / "out"
    rc = optimize.main(["--output-dir", str(out), "--device", "cpu", "--batch-size", "1", "--seq-len", "4",
                        "--hidden-dim", "64", "--num-heads", "4", "--head-dim", "16", "--ffn-dim", "96",
                        "--dtype", "fp32", "--cache-path", str(tmp_path / "c.json")])
    assert rc == 0
    doc = json.loads((out / "selected_config.json").read_text())
    assert set(doc) == {"gpu", "compute_backend", "device", "created_at", "parameters", "operations", "cache"}
    assert set(doc["operations"]) == {"rmsnorm", "rmsnorm_residual", "rope", "rope_qk", "swiglu"}
    assert doc["parameters"]["hidden_dim"] == 64 and doc["parameters"]["dtype"] == "float32"
    for op in doc["operations"].values():
        assert op["source"] == "default" and op["selected_kernel"]
    assert doc["compute_backend"] == "cpu"
    lines = optimize.summary_lines(doc)
    assert len(lines) == 5 and "[default]" in lines[0]


def test_environment_report_on_the_cpu(capsys) -> None:
    """The ``check_environment`` equivalent: runtime versions, device, whether
    the library and binding load; exit 0 on a CPU-only machine."""
    state = env.report()
    assert state["torch"] == torch.__version__ and state["gpu_available"] is False
    assert state["compute_backend"] == "cpu" and state["cache_key"] == "cpu_-1"
    assert "arch=gfx950" in state["hip_library"] or state["hip_library"].startswith("not loadable")
    assert env.main([]) == 0
    out = capsys.readouterr().out
    assert "hip_library" in out and "CPU only" in out


def _two_cards(tmp_path):
    """A DRM tree with card2 and card10 (card10 sorts first as a string), each
    with its PCI address, clock levels and load, and a KFD tree with a CPU node
    and both GPU nodes."""
    drm = tmp_path / "drm"
    for card, slot, busy, sclk in (("card2", "0000:5a:00.0", "0", "0: 500Mhz *\n1: 2400Mhz\n"),
                                   ("card10", "0000:c3:00.0", "80", "0: 500Mhz\n1: 2200Mhz *\n")):
        dev = drm / card / "device"
        dev.mkdir(parents=True)
        (dev / "uevent").write_text(f"DRIVER=amdgpu\nPCI_CLASS=12000\nPCI_SLOT_NAME={slot}\n")
        (dev / "gpu_busy_percent").write_text(busy + "\n")
        (dev / "pp_dpm_sclk").write_text(sclk)
    (drm / "card2-DP-1").mkdir()  # connectors are not cards
    topo = tmp_path / "topology"
    for node, gpu_id, location in (("0", "0", 0), ("1", "28206", 0x5A00), ("2", "41733", 0xC300)):
        (topo / node).mkdir(parents=True)
        (topo / node / "gpu_id").write_text(gpu_id + "\n")
        (topo / node / "properties").write_text(f"cpu_cores_count 0\nlocation_id {location}\ndomain 0\n")
    kfd = tmp_path / "kfd_proc"
    for pid, entries in ((os.getpid(), ["vram_28206", "queues"]), (4242, ["vram_41733", "sdma_41733"]),
                         (5151, ["queues"])):
        for e in entries:
            (kfd / str(pid) / e).mkdir(parents=True)
    return drm, topo, kfd


def test_cards_are_matched_by_pci_address(tmp_path) -> None:
    """Cards sort by number (card2 before card10); a PCI address picks its
    card whatever its position; the peak clock is the highest sclk level,
    not the active one; the KFD node is found by domain and location id."""
    from ako_amd.dispatcher import amdgpu_sysfs as sysfs

    drm, topo, _ = _two_cards(tmp_path)
    assert [d.parent.name for d in sysfs.card_device_dirs(drm)] == ["card2", "card10"]
    assert sysfs.device_dir(1, drm=drm, slot="0000:5A:00.0").parent.name == "card2"
    assert sysfs.device_dir(0, drm=drm, slot="0000:c3:00.0").parent.name == "card10"
    assert sysfs.device_dir(0, drm=drm, slot="0000:01:00.0") is None
    assert sysfs.peak_sclk_khz(drm / "card2" / "device") == 2_400_000
    assert sysfs.peak_sclk_khz(drm / "card10" / "device") == 2_200_000
    assert sysfs.pci_slot_name(0, 0x5A, 0) == "0000:5a:00.0"
    assert sysfs.kfd_gpu_id("0000:5a:00.0", topo) == 28206
    assert sysfs.kfd_gpu_id("0000:c3:00.0", topo) == 41733
    assert sysfs.kfd_gpu_id("0000:77:00.0", topo) is None
    # Without torch's PCI address (no GPU here) the index is the card-number position.
    assert sysfs.device_dir(1, drm=drm).parent.name == "card10"


def test_preflight_looks_at_its_own_card(tmp_path) -> None:
    """The idle card2 with only this process on it passes even though card10
    is busy and another process holds a context there; card10 is refused for
    its load and its process; a process with no per-GPU entries counts on
    both."""
    drm, topo, kfd = _two_cards(tmp_path)
    state = env.preflight(0, drm=drm, kfd_proc=kfd, topology=topo, slot="0000:5a:00.0", strict=False)
    assert state["utilization_gpu"] == 0.0 and state["compute_apps"] == [5151]
    state = env.preflight(0, drm=drm, kfd_proc=kfd, topology=topo, slot="0000:c3:00.0", strict=False)
    assert state["busy"] and state["utilization_gpu"] == 80.0 and state["compute_apps"] == [4242, 5151]
    # An unknown node: every process counts.
    assert env.gpu_processes(kfd) == sorted([os.getpid(), 4242, 5151])
    sample = env.sample_env(0, drm=drm, slot="0000:c3:00.0")
    assert sample["sm_clock_mhz"] == 2200.0
