"""Build ``libako_hip.so`` (the C-ABI kernel library) for gfx950 with hipcc.

The library is linked against the HIP runtime that PyTorch-ROCm ships in
``torch/lib`` (``libamdhip64.so``, SONAME ``libamdhip64.so.7``), not against
``/opt/rocm/lib``: once ``torch`` is imported, the dynamic loader resolves the
library's HIP dependency to the runtime torch already loaded, so device
pointers and ``hipStream_t`` handles handed over from torch belong to the same
runtime instance. ``ako_amd._native`` verifies that at load time.

Flags that matter:
  -ffp-contract=off         products and sums are rounded one at a time, as in
                            the unfused PyTorch references;
  -packed-fp32-ops (off)    no v_pk_*_f32 instructions are generated;
  -mcode-object-version=5   loadable by every ROCm 6.x/7.x runtime.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libako_hip.so"
OBJ_DIR = LIB_DIR / "_build"
SOURCES = ("abi.hip", "rmsnorm.hip", "rope.hip", "swiglu.hip")
ARCH = "gfx950"


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found (expected on PATH or /opt/rocm/bin)")
    return found


def torch_lib_dir() -> Path:
    import torch

    return Path(torch.__file__).resolve().parent / "lib"


def compile_flags(extra: list[str] | None = None) -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-mcode-object-version=5",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        *(extra or []),
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; harmless.
    noise = ("packed-fp32-ops", "warning generated when compiling for host", "warnings generated when compiling for host")
    text = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if not any(n in line for n in noise)
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{text}")
    if text and verbose:
        print(text, flush=True)


def build_library(*, verbose: bool = False, extra_flags: list[str] | None = None,
                  output: Path | None = None) -> Path:
    """Compile every kernel source and link ``libako_hip.so``; returns its path."""
    hipcc = _hipcc()
    out = Path(output) if output is not None else LIB_PATH
    obj_dir = OBJ_DIR if output is None else out.parent / f"_build_{out.stem}"
    obj_dir.mkdir(parents=True, exist_ok=True)
    flags = compile_flags(extra_flags)
    objects = [obj_dir / (Path(src).stem + ".o") for src in SOURCES]
    jobs = [[hipcc, *flags, "-c", str(CSRC / src), "-o", str(obj)] for src, obj in zip(SOURCES, objects)]
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "4")), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda cmd: _run(cmd, verbose), jobs))
    tlib = torch_lib_dir()
    tmp = out.with_name(out.name + f".tmp{os.getpid()}")
    link = [
        hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp),
        f"-L{tlib}", "-lamdhip64", f"-Wl,-rpath,{tlib}",
    ]
    _run(link, verbose)
    os.replace(tmp, out)
    return out


BINDING_SOURCE = CSRC / "torch_bind.cpp"


def binding_path() -> Path:
    import sysconfig

    return LIB_DIR / ("_ako_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_torch_binding(*, verbose: bool = False) -> Path:
    """Compile the PyTorch binding (``_ako_torch``, host code only, g++).

    It links ``libako_hip.so`` from the same directory (rpath ``$ORIGIN``)
    and torch's libraries; the HIP headers are needed only for torch's HIP
    stream API. Build the kernel library first.
    """
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} must be built before the torch binding")
    try:
        includes = cpp_extension.include_paths(device_type="cuda")
    except TypeError:  # older signature
        includes = cpp_extension.include_paths(cuda=True)
    tlib = torch_lib_dir()
    out = binding_path()
    tmp = out.with_name(out.name + f".tmp{os.getpid()}")
    abi = int(bool(getattr(torch._C, "_GLIBCXX_USE_CXX11_ABI", True)))
    cmd = [
        shutil.which("g++") or "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_ako_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-I{INCLUDE}", f"-I{sysconfig.get_paths()['include']}",
        *(f"-I{p}" for p in includes), "-I/opt/rocm/include",
        str(BINDING_SOURCE), "-o", str(tmp),
        f"-L{LIB_DIR}", "-lako_hip", "-Wl,-rpath,$ORIGIN",
        f"-L{tlib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
        "-lamdhip64", f"-Wl,-rpath,{tlib}",
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


COPY_PROBE_SOURCE = PACKAGE_DIR / "benchmark" / "copy_ceiling.hip"
COPY_PROBE_PATH = LIB_DIR / "copy_ceiling"


def build_copy_probe(*, verbose: bool = False) -> Path:
    """Compile the stand-alone copy-ceiling program (size-dependent HBM ceiling)."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = COPY_PROBE_PATH.with_name(COPY_PROBE_PATH.name + f".tmp{os.getpid()}")
    _run([_hipcc(), *compile_flags(), str(COPY_PROBE_SOURCE), "-o", str(tmp)], verbose)
    os.replace(tmp, COPY_PROBE_PATH)
    return COPY_PROBE_PATH


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
    print(build_torch_binding(verbose="-v" in sys.argv))
    print(build_copy_probe(verbose="-v" in sys.argv))
