"""ctypes binding of ``libako_hip.so`` (declared in ``include/ako_hip.h``).

Loading is lazy and happens once. It fails loudly: a missing or mismatched
library raises ``HipLibraryError`` rather than letting any caller fall back
to a CPU or PyTorch path. Two checks run at load time:

* the ABI version compiled into the library equals ``ABI_VERSION``;
* the HIP runtime the library is bound to is the one PyTorch uses
  (``hipRuntimeGetVersion`` against ``torch.version.hip``). The library is
  linked against torch's bundled ``libamdhip64``; if some other runtime were
  resolved, device pointers and stream handles from torch would belong to a
  different runtime instance.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Any

import torch

ABI_VERSION = 1
LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libako_hip.so"

AKO_OK = 0
AKO_ERR_INVALID_ARGUMENT = 1
AKO_ERR_UNSUPPORTED = 2
AKO_ERR_HIP = 3
AKO_ERR_NO_DEVICE = 4

DTYPE_CODES: dict[torch.dtype, int] = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
ROPE_STYLE_CODES = {"neox": 0, "interleaved": 1}

#: Every symbol the header declares, with its (restype, argtypes).
_i64, _int, _ptr, _f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "ako_abi_version": (_int, []),
    "ako_hip_runtime_version": (_int, []),
    "ako_build_info": (ctypes.c_char_p, []),
    "ako_last_error": (ctypes.c_char_p, []),
    "ako_device_identity": (_int, [_int, ctypes.c_char_p, _i64]),
    "ako_rmsnorm_fwd": (_int, [_ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _f32, _int, _int, _ptr]),
    "ako_rmsnorm_residual_fwd": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _ptr],
    ),
    "ako_rmsnorm_shard_partial_fwd": (_int, [_ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _int, _ptr]),
    "ako_rmsnorm_shard_apply_fwd": (
        _int, [_ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _ptr],
    ),
    "ako_rope_fwd": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _int, _int, _int, _ptr],
    ),
    # The four stride arguments are `const int64_t*`; they are passed as
    # addresses into one ctypes array (c_void_p) to keep the call cheap.
    "ako_rope_qk_fwd": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr,
         _ptr, _i64, _int, _int, _int, _ptr],
    ),
    "ako_rope_qk_cache_fwd": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64,
         _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _int, _int, _int, _ptr],
    ),
    "ako_swiglu_fwd": (_int, [_ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _int, _ptr]),
    "ako_set_tuning": (_int, [_int, _int, _int]),
    "ako_time_next_launch": (_int, [_ptr, _ptr]),
}


class HipLibraryError(RuntimeError):
    """The HIP kernel library is missing, stale, or bound to the wrong runtime."""


_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.environ.get("AKO_HIP_LIB")
    return Path(override) if override else LIB_PATH


def _expected_runtime_version() -> int | None:
    """``torch.version.hip`` ("7.0.51831") as hipRuntimeGetVersion encodes it."""
    text = getattr(torch.version, "hip", None)
    if not text:
        return None
    parts = [int(p) for p in text.split(".")[:3] if p.isdigit()]
    while len(parts) < 3:
        parts.append(0)
    major, minor, patch = parts
    return major * 10_000_000 + minor * 100_000 + patch


def load() -> ctypes.CDLL:
    """The loaded library; raises ``HipLibraryError`` when it cannot be used."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise HipLibraryError(
            f"{path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or `python -m ako_amd._build`) first"
        )
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as exc:
        raise HipLibraryError(f"cannot load {path}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            raise HipLibraryError(f"{path} does not export {name}")
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.ako_abi_version() != ABI_VERSION:
        raise HipLibraryError(
            f"{path} has ABI {lib.ako_abi_version()}, this package needs {ABI_VERSION}; rebuild it"
        )
    expected = _expected_runtime_version()
    bound = lib.ako_hip_runtime_version()
    if expected is not None and bound != expected:
        raise HipLibraryError(
            f"{path} is bound to HIP runtime {bound}, but torch uses {expected} "
            f"({torch.version.hip}); the library must link torch's libamdhip64"
        )
    _lib = lib
    return lib


_binding: Any = None
_binding_checked = False


def torch_binding() -> Any:
    """The PyTorch binding module ``_ako_torch`` (built next to the library by
    ``ako_amd._build.build_torch_binding``), or ``None`` when it is not built
    or ``AKO_TORCH_BINDING=0``.

    It does each HIP candidate's host work (checks, allocation, stream) in
    C++ and calls the same C ABI; without it the candidates make the same
    calls through ctypes. Both launch the same kernels of this library: the
    binding is a faster host path, never a different compute path. Loading
    it loads (and checks) the kernel library first.
    """
    global _binding, _binding_checked
    if _binding_checked:
        return _binding
    _binding_checked = True
    if os.environ.get("AKO_TORCH_BINDING", "1").strip() == "0":
        return None
    load()
    import importlib.util
    import logging
    import sysconfig

    path = library_path().with_name("_ako_torch" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not path.exists():
        return None
    try:
        spec = importlib.util.spec_from_file_location("_ako_torch", path)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
    except ImportError as exc:
        logging.getLogger(__name__).warning("torch binding %s not usable (%s); using ctypes", path, exc)
        return None
    if module.abi_version() != ABI_VERSION:
        raise HipLibraryError(f"{path} was built for ABI {module.abi_version()}, need {ABI_VERSION}; rebuild")
    _binding = module
    return module


def is_available() -> bool:
    try:
        load()
    except HipLibraryError:
        return False
    return True


def last_error() -> str:
    raw = load().ako_last_error()
    return raw.decode() if raw else ""


def check(status: int, fn_name: str) -> None:
    """Turn a nonzero ``ako_status_t`` into the reference's exception types."""
    if status == AKO_OK:
        return
    message = f"{fn_name}: {last_error()}"
    if status in (AKO_ERR_INVALID_ARGUMENT, AKO_ERR_UNSUPPORTED):
        raise ValueError(message)
    raise RuntimeError(message)


def set_tuning(op: int, key: int, value: int) -> None:
    check(load().ako_set_tuning(op, key, value), "ako_set_tuning")


def time_next_launch(start: "torch.cuda.Event", stop: "torch.cuda.Event") -> None:
    """Bind ``start`` and ``stop`` to the next kernel launch this thread makes
    through the library (``ako_time_next_launch``): their elapsed time is then
    that kernel's own duration. Each event must have been recorded once
    before, so that torch has created it."""
    handles = (int(start.cuda_event), int(stop.cuda_event))
    if not all(handles):
        raise ValueError("time_next_launch: record each event once before arming it")
    check(load().ako_time_next_launch(*handles), "ako_time_next_launch")


def disarm_launch_timing() -> bool:
    """Drop an armed event pair; True when one was still armed (no launch took it)."""
    status = load().ako_time_next_launch(None, None)
    if status not in (0, 1):
        check(status, "ako_time_next_launch")
    return status == 1


def current_stream(device: torch.device) -> int:
    """Raw ``hipStream_t`` of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def device_identity(index: int) -> dict[str, str]:
    """HIP's identity fields of GPU ``index`` (``ako_device_identity``) as a dict."""
    buf = ctypes.create_string_buffer(1024)
    check(load().ako_device_identity(int(index), buf, len(buf)), "ako_device_identity")
    fields = {}
    for item in buf.value.decode(errors="replace").split(";"):
        key, _, value = item.partition("=")
        fields[key] = value
    return fields
