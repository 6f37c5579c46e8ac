"""Binding of the C-ABI HIP library (lib/libgs3d_hip.so) through ctypes.

This replaces the Warp launch path of the reference (runtime/dispatch.py:
184-237 ``launch``/``launch_tiled`` with their descriptor and command caches):
every kernel entry point takes raw device pointers, sizes and the current
HIP stream, so there is nothing to cache on the host besides the library
handle.  There is no fallback: if the library is absent or the process has
no HIP device, the call raises.
"""

import ctypes
import functools
import os
import threading

import torch

from . import abi

_LIB_PATH = os.environ.get(
    "GS3D_HIP_LIBRARY",
    os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib", "libgs3d_hip.so"),
)
_lock = threading.Lock()
_lib = None


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, stale or returned an error status."""


def library_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load and type the library (idempotent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise NativeLibraryError(
                f"{_LIB_PATH} is missing: build it with `python -m dsl_splat_amd.build` "
                "(hipcc, gfx950); there is no non-HIP fallback"
            )
        lib = ctypes.CDLL(_LIB_PATH)
        for name, (restype, argtypes) in abi.FUNCTIONS.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.gs3d_abi_version()
        if version != abi.ABI_VERSION:
            raise NativeLibraryError(
                f"{_LIB_PATH} has ABI version {version}, expected {abi.ABI_VERSION}; rebuild it"
            )
        _lib = lib
    return _lib


def check(status: int, name: str) -> None:
    if status != abi.GS3D_OK:
        detail = load().gs3d_last_error().decode(errors="replace")
        kind = abi.STATUS_NAMES.get(status, f"status {status}")
        raise NativeLibraryError(f"{name} failed: {kind}" + (f" ({detail})" if detail else ""))


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


# torch's raw current-stream lookup (one C call) where this torch has it;
# torch.cuda.current_stream builds a Stream object on every call (~6 us of
# host time, several times per rasterize).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device: torch.device) -> ctypes.c_void_p:
    """Handle of torch's current stream on ``device`` (the launch stream)."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return ctypes.c_void_p(_raw_stream(index))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(tensor: torch.Tensor | None, offset_elems: int = 0) -> int | None:
    """Device address of a tensor's first element (plus an element offset),
    as the integer that ctypes passes for a ``void*`` argument or field."""
    if tensor is None:
        return None
    if offset_elems:
        return tensor.data_ptr() + offset_elems * tensor.element_size()
    return tensor.data_ptr()


def no_grad(fn):
    """torch.no_grad() as a decorator that costs nothing when gradients are
    already off (the launch wrappers call one another; torch's decorator
    enters a fresh context manager on every call)."""

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        if not torch.is_grad_enabled():
            return fn(*args, **kwargs)
        with torch.no_grad():
            return fn(*args, **kwargs)

    return wrapper


def require_device(tensor: torch.Tensor) -> None:
    if not isinstance(tensor, torch.Tensor) or tensor.device.type != "cuda":
        raise ValueError("gs3d kernels need tensors on a HIP device (torch 'cuda' device)")
