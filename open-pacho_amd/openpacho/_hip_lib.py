"""ctypes binding of libpacho_hip.so (declared in include/pacho_hip.h).

The library is looked up at ``PACHO_HIP_LIBRARY`` or next to this module.
Nothing here initialises the GPU: loading the shared object only resolves
symbols. Status codes map to Python exceptions with the library's message.
"""

import ctypes
import os
import threading
from pathlib import Path

import numpy as np

from .exceptions import BackendUnavailableError

LIBRARY_NAME = "libpacho_hip.so"

HP_OK, HP_E_INVALID, HP_E_HIP, HP_E_OOM, HP_E_RTC, HP_E_UNSUPPORTED, HP_E_INJECTED = range(7)
DTYPE_CODES = {
    np.dtype("bool"): 0,
    np.dtype("int32"): 1,
    np.dtype("int64"): 2,
    np.dtype("uint32"): 3,
    np.dtype("uint64"): 4,
    np.dtype("float32"): 5,
    np.dtype("float64"): 6,
}
DISTRIBUTIONS = {"random": 0, "uniform": 1, "normal": 2, "exponential": 3}
REDUCTIONS = {"sum": 0, "min": 1, "max": 2}

_i32, _i64, _u32, _u64 = ctypes.c_int, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64
_ptr, _pptr, _cstr = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> argument types (every function returns int unless listed in _RESTYPES)
PROTOTYPES = {
    "hp_last_error": [],
    "hp_version": [],
    "hp_device_count": [ctypes.POINTER(ctypes.c_int)],
    "hp_device_info": [_i32, _cstr, _i64, _cstr, _i64, _i64p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)],
    "hp_init": [_i32, _pptr],
    "hp_destroy": [_ptr],
    "hp_alloc": [_ptr, _i64, _pptr],
    "hp_free": [_ptr, _ptr],
    "hp_release_cached": [_ptr],
    "hp_set_pool_limit": [_ptr, _i64],
    "hp_pool_stats": [_ptr, _i64p, _i64p, _i64p, _i64p],
    "hp_h2d": [_ptr, _ptr, _ptr, _i64],
    "hp_d2h": [_ptr, _ptr, _ptr, _i64],
    "hp_d2d": [_ptr, _ptr, _ptr, _i64],
    "hp_sync": [_ptr],
    "hp_fill": [_ptr, _ptr, _i64, _i32, _u64],
    "hp_gather": [_ptr, _i32, _ptr, _ptr, _i64, _i32, _i64p, _i64p],
    "hp_pad_copy": [_ptr, _i32, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64],
    "hp_gemm": [_ptr, _i32, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i32, _i64p, _i64p, _i64p],
    "hp_gemm_layout": [_ptr, _i32, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i32, _i32],
    "hp_gemv": [_ptr, _i32, _ptr, _ptr, _ptr, _i64, _i64],
    "hp_gemv_residual": [_ptr, _i32, _ptr, _ptr, _ptr, _ptr, _i64, _i64],
    "hp_dot": [_ptr, _i32, _ptr, _ptr, _ptr, _i64],
    "hp_dot_new": [_ptr, _i32, _ptr, _ptr, _i64, _pptr],
    "hp_norm": [_ptr, _i32, _ptr, _ptr, _i64, _i64, _i64],
    "hp_norm_noalloc": [_ptr, _i32, _ptr, _ptr, _i64, _i64, _i64],
    "hp_reduce": [_ptr, _i32, _i32, _ptr, _ptr, _i64, _i64, _i64],
    "hp_philox": [_ptr, _i32, _i32, _ptr, _i64, _u64, _u64, ctypes.c_double, ctypes.c_double, ctypes.c_double],
    "hp_philox_words": [_ptr, _ptr, _i64, _u64, _u64],
    "hp_rtc_compile": [_ptr, _cstr, _cstr, _pptr],
    "hp_rtc_launch": [_ptr, _ptr, _i64, _i32, _i32, _pptr],
    "hp_rtc_release": [_ptr, _ptr],
    "hp_event_create": [_ptr, _pptr],
    "hp_event_record": [_ptr, _ptr],
    "hp_event_elapsed_ms": [_ptr, _ptr, ctypes.POINTER(ctypes.c_float)],
    "hp_event_destroy": [_ptr],
    "hp_debug_fail_next": [_ptr, _i32],
}
_RESTYPES = {"hp_last_error": ctypes.c_char_p, "hp_version": ctypes.c_char_p}

_lock = threading.Lock()
_library = None


def library_path():
    override = os.environ.get("PACHO_HIP_LIBRARY")
    return Path(override) if override else Path(__file__).resolve().with_name(LIBRARY_NAME)


def load():
    """Load and type the shared library once per process."""
    global _library
    with _lock:
        if _library is not None:
            return _library
        path = library_path()
        if not path.exists():
            raise BackendUnavailableError(
                f"{LIBRARY_NAME} not found at {path}; build it with `python open-pacho_amd/build.py`"
            )
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            raise BackendUnavailableError(f"Cannot load {path}: {exc}") from exc
        for name, argtypes in PROTOTYPES.items():
            function = getattr(lib, name)
            function.argtypes = argtypes
            function.restype = _RESTYPES.get(name, ctypes.c_int)
        _library = lib
        return lib


def last_error(lib):
    message = lib.hp_last_error()
    return message.decode(errors="replace") if message else ""


def check(lib, status, what):
    """Raise the Python exception for a nonzero status."""
    if status == HP_OK:
        return
    message = f"{what}: {last_error(lib)}"
    if status == HP_E_INVALID:
        raise ValueError(message)
    if status == HP_E_UNSUPPORTED:
        raise NotImplementedError(message)
    # Driver failures, including out-of-memory, are RuntimeErrors as in the
    # reference's CUDA backend (_cuda.py:49-53).
    raise RuntimeError(f"HIP call failed ({status}): {message}")


def int64_array(values):
    values = list(values)
    return (ctypes.c_int64 * max(1, len(values)))(*values)
