"""ctypes binding of liblynnreal_amd.so, the gfx950 C ABI (include/lynnreal_amd.h).

The library is loaded lazily on first use. There is no fallback: if the
library is missing or the device is not a gfx950 GPU, every call raises.

Status codes map to the exception types the reference's error policy expects
(model/acceleration.py:49-56 treats "not supported" messages as recoverable
and never recovers from out-of-memory):
  LR_EINVAL       -> ValueError
  LR_EUNSUPPORTED -> RuntimeError("... not supported")
  LR_ENOMEM       -> torch.cuda.OutOfMemoryError
  LR_EHIP         -> RuntimeError
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch

LIBRARY = pathlib.Path(__file__).resolve().parent / "liblynnreal_amd.so"

LR_OK, LR_EINVAL, LR_EUNSUPPORTED, LR_EHIP, LR_ENOMEM = 0, 1, 2, 3, 4
EPI_BF16, EPI_GELU_TANH, EPI_GATED_RESIDUAL, EPI_RAW_INT32 = 0, 1, 2, 3
DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2
(TILE_AUTO, TILE_256x256, TILE_256x128, TILE_128x256, TILE_128x128, TILE_64x128, TILE_GENERIC,
 TILE_256x256_W4x2, TILE_256x192, TILE_256x80, TILE_64x80, TILE_128x160, TILE_192x256,
 TILE_256x256_PERSISTENT) = range(14)
ABI_VERSION = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

# name -> argument types (every entry point returns int).
SIGNATURES = {
    "lr_quantize_rows": [_P, _I64, _I64, _P, _P, _P],
    "lr_quantize_rows_typed": [_P, _I32, _I64, _I64, _P, _P, _P],
    "lr_int8_gemm": [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I32, _P, _P, _I64,
                     _I64, _P, _I64, _I32, _I32, _P],
    "lr_int8_gemm_ws": [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I32, _P, _P, _I64,
                        _I64, _P, _I64, _I32, _P, _I64, _I32, _I32, _P],
    "lr_int8_gemm_noalloc": [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I32, _P, _P, _I64,
                             _I64, _P, _I64, _I32, _I32, _I32, _P],
    "lr_int8_epilogue": [_P, _P, _P, _P, _P, _I64, _I64, _P],
    "lr_rms_adaln": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _F32, _P],
    "lr_rms_adaln_quant": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32,
                           _F32, _P],
    "lr_residual_rms_quant": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                              _F32, _P],
    "lr_gated_residual": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P],
    "lr_swiglu": [_P, _P, _I64, _I64, _P],
    "lr_swiglu_quant": [_P, _P, _P, _I64, _I64, _P],
    "lr_gelu_tanh": [_P, _P, _I64, _P],
    "lr_gelu_quant": [_P, _P, _P, _I64, _I64, _P],
    "lr_qk_norm_rope": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                        _I64, _I64, _F32, _P],
    "lr_gather_rows": [_P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "lr_flash_restore": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P],
    "lr_flash_nearest_anchor": [_P, _I64, _P, _I64, _P, _I64, _P, _P],
    "lr_adaln_table": [_P, _I32, _I32, _P, _P, _P, _I64, _I64, _I64, _P],
    "lr_device_supported": [_I32],
    "lr_abi_version": [],
}

_lock = threading.Lock()
_lib = None


def library_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get("LYNNREAL_AMD_LIBRARY", LIBRARY))


def load() -> ctypes.CDLL:
    """Load the HIP library (once) and declare its prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python -m lynnreal_omni_amd.build` "
                "(the W8A8 path has no CPU fallback)")
        lib = ctypes.CDLL(str(path))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        lib.lr_last_error.argtypes = []
        lib.lr_last_error.restype = ctypes.c_char_p
        lib.lr_int8_gemm_workspace_size.argtypes = [_I64, _I64, _I64, _I32, _I32]
        lib.lr_int8_gemm_workspace_size.restype = ctypes.c_int64
        if lib.lr_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI {lib.lr_abi_version()}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def raise_for(status: int, name: str) -> None:
    if status == LR_OK:
        return
    message = f"{name}: {load().lr_last_error().decode(errors='replace')}"
    if status == LR_EINVAL:
        raise ValueError(message)
    if status == LR_EUNSUPPORTED:
        raise RuntimeError(message if "not supported" in message else message + " (not supported)")
    if status == LR_ENOMEM:
        raise torch.cuda.OutOfMemoryError(message)
    raise RuntimeError(message)


try:
    from . import _pycall
except ImportError:  # not built: every call goes through ctypes
    _pycall = None

_entry: dict[str, object] = {}


def _bind(name: str):
    """The callable for entry point `name`: the _pycall fast call with the
    function's address when every argument is a pointer or an integer, else
    the ctypes function (entry points with float arguments)."""
    fn = getattr(load(), name)
    if _pycall is not None and all(t in (_P, _I64, _I32) for t in SIGNATURES[name]):
        address = ctypes.cast(fn, ctypes.c_void_p).value
        fast = _pycall.call
        return lambda *args: fast(address, *args)
    return fn


def call(name: str, *args) -> None:
    """Call entry point `name` and raise on a non-zero status."""
    fn = _entry.get(name)
    if fn is None:
        fn = _entry[name] = _bind(name)
    status = fn(*args)
    if status:
        raise_for(status, name)


_checked_devices: dict[int, bool] = {}


def check_device(t: torch.Tensor) -> None:
    """Raise unless `t` lives on a gfx950 GPU the library supports."""
    if not t.is_cuda:
        raise ValueError(f"the W8A8 HIP path needs GPU tensors, got a tensor on {t.device}")
    index = t.get_device()
    ok = _checked_devices.get(index)
    if ok is None:
        ok = _checked_devices[index] = bool(load().lr_device_supported(index))
    if not ok:
        raise RuntimeError(f"device {index} ({torch.cuda.get_device_name(index)}) is not supported: "
                           "liblynnreal_amd.so is built for gfx950 only")


def same_device(primary: torch.Tensor, **tensors) -> None:
    """Raise ValueError unless every tensor given (None is skipped) lives on
    `primary`'s device. The kernels receive raw pointers, so a host tensor or
    one on another GPU must be refused here, before any launch."""
    index = primary.get_device()
    for t in tensors.values():
        if t is not None and t.get_device() != index:
            name = next(k for k, v in tensors.items() if v is t)
            raise ValueError(f"{name} is on {t.device}, but the kernel runs on {primary.device}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(t: torch.Tensor) -> int:
    """The caller's current HIP stream on t's device (Triton's launch behaviour)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_MAX_WORKSPACES = 16


def workspace(t: torch.Tensor, nbytes: int) -> tuple[int | None, int]:
    """(pointer, bytes) of a device workspace of at least `nbytes` for the
    caller's current stream on t's device, or (None, 0) when none is needed.

    One buffer is kept per (device, stream), grown on demand, for the 16
    most recently used (device, stream) pairs: kernels that share a buffer
    run in stream order, and torch's caching allocator hands a released
    buffer's memory to a later allocation on the same stream only, behind
    the work already queued there."""
    if nbytes <= 0:
        return None, 0
    key = (t.get_device(), stream(t))
    buf = _workspaces.pop(key, None)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(nbytes, dtype=torch.uint8, device=t.device)
    _workspaces[key] = buf  # most recent last
    while len(_workspaces) > _MAX_WORKSPACES:
        _workspaces.pop(next(iter(_workspaces)))
    return buf.data_ptr(), buf.numel()
