"""ctypes binding of libjeeves_fp8.so (the C ABI in include/jeeves_fp8.h).

The library is loaded from this package's directory only: the FP8 path has no
CPU or PyTorch fallback, so a missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libjeeves_fp8.so")

JV_OK, JV_ERR_VALUE, JV_ERR_RUNTIME, JV_ERR_HIP = 0, 1, 2, 3

# name -> (restype, argtypes); mirrors include/jeeves_fp8.h
SIGNATURES: dict[str, tuple] = {
    "jv_fp8_last_error": (c_char_p, []),
    "jv_device_cu_count": (c_int, [c_int]),
    "jv_fp8_quantize_rows_bf16": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "jv_fp8_quantize_rows_f32": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "jv_fp8_quantize_rows_host": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int]),
    "jv_fp8_packed_codes_bytes": (c_int64, [c_int64, c_int64]),
    "jv_fp8_linear_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64]),
    "jv_fp8_linear": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_float,
                              c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, POINTER(c_int32), c_int64,
                              c_void_p]),
    "jv_fp8_linear_noalloc": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                      c_float, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "jv_fp8_gemm_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "jv_fp8_gemm": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                            c_float, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, POINTER(c_int32), c_int64,
                            c_void_p]),
    "jv_fp8_swiglu_quantize": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                                       c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "jv_fp8_linear_swiglu": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                     c_float, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64,
                                     POINTER(c_int32), c_int64, c_void_p]),
    "jv_fp8_quantize_swiglu_output": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                                              c_void_p, c_int64, c_void_p, c_void_p]),
    "jv_w8a16_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "jv_w8a16_linear": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64,
                                c_int64, c_void_p, c_int64, POINTER(c_int32), c_int64, c_void_p]),
    "jv_fp8_tile_weight": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "jv_fp8_untile_weight": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "jv_fp8_split_for": (c_int, [c_int64, c_int64, c_int64, c_int]),
    "jv_fp8_counters_needed": (c_int64, [c_int64, c_int64, c_int64, c_int]),
    "jv_fp8_launch_shape": (c_int, [c_int64, c_int64, c_int64, c_int, POINTER(c_int32)]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """The loaded library with typed entry points (loaded once)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(f"{LIB_PATH.name} is not built: run `python -m jeeves_amd.build` (needs hipcc)")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype, fn.argtypes = res, args
                _lib = handle
    return _lib


def check(rc: int) -> None:
    """Map a JV_* status to the exception the reference raises for that case."""
    if rc == JV_OK:
        return
    msg = lib().jv_fp8_last_error().decode(errors="replace")
    if rc == JV_ERR_VALUE:
        raise ValueError(msg)
    raise RuntimeError(msg)


def counters_ptr(t) -> "ctypes._Pointer":
    return ctypes.cast(c_void_p(t.data_ptr()), POINTER(c_int32)) if t is not None else None
