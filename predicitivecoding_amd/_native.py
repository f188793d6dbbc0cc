"""ctypes binding of libpcdevice_hip.so (the C ABI in include/pcdevice.h).

The library is the only compute path: if it is missing this module raises
instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os
import re

from .errors import DeviceException

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpcdevice_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "pcdevice.h")

_lib = None

c_int, c_float, c_size_t, c_void_p, c_char_p = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
P_int = ctypes.POINTER(ctypes.c_int)
P_float = ctypes.POINTER(ctypes.c_float)
P_void_p = ctypes.POINTER(ctypes.c_void_p)

_SIGNATURES = {
    "pcd_get_device_count": [P_int],
    "pcd_set_device": [c_int],
    "pcd_get_device": [P_int],
    "pcd_device_synchronize": [],
    "pcd_last_error": [c_char_p, c_size_t],
    "pcd_version": [P_int],
    "pcd_malloc_async": [P_void_p, c_size_t, c_void_p],
    "pcd_free_async": [c_void_p, c_void_p],
    "pcd_host_alloc": [P_void_p, c_size_t],
    "pcd_host_free": [c_void_p],
    "pcd_trim_pools": [],
    "pcd_memcpy": [c_void_p, c_void_p, c_size_t, c_int],
    "pcd_memcpy_async": [c_void_p, c_void_p, c_size_t, c_int, c_void_p],
    "pcd_memset_async": [c_void_p, c_int, c_size_t, c_void_p],
    "pcd_stream_create": [P_void_p],
    "pcd_stream_destroy": [c_void_p],
    "pcd_stream_synchronize": [c_void_p],
    "pcd_event_create": [P_void_p],
    "pcd_event_record": [c_void_p, c_void_p],
    "pcd_event_synchronize": [c_void_p],
    "pcd_event_destroy": [c_void_p],
    "pcd_event_elapsed_ms": [P_float, c_void_p, c_void_p],
    "pcd_gemm_f32": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p],
    "pcd_gemm_bf16": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p],
    "pcd_gemm_f16": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p],
    "pcd_gemm_f32_batched": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p],
    "pcd_gemm_bf16_batched": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p],
    "pcd_gemm_f16_batched": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p],
    "pcd_pc_model_create": [P_int, c_int, c_int, c_float, c_float, c_int, P_void_p, P_void_p, P_float, c_int, P_void_p],
    "pcd_pc_model_destroy": [c_void_p],
    "pcd_pc_relax": [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p],
    "pcd_pc_relax_noalloc": [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p],
    "pcd_pc_relax_ragged": [c_void_p, c_void_p, P_int, P_int, c_int, c_int, c_float, P_int, c_void_p, P_float, c_void_p],
    "pcd_pc_relax_clamped": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p],
    "pcd_pc_classify": [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p],
    "pcd_pc_classify_adaptive": [c_void_p, c_void_p, c_int, c_int, c_float, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_void_p],
    "pcd_pc_learn": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_float, c_void_p, c_void_p],
    "pcd_pc_learn_warm": [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_float, c_void_p,
                          c_void_p],
    "pcd_pc_model_get_weights": [c_void_p, c_int, c_void_p, c_void_p],
    "pcd_pc_model_load_record": [c_void_p, c_int, c_void_p, c_size_t],
    "pcd_pc_model_info": [c_void_p, P_int, P_int, c_int, P_int],
    "pcd_pc_set_option": [c_void_p, c_char_p, c_int],
    "pcd_pc_profile_result": [c_void_p, P_float, P_float, P_int],
}

# enum values of include/pcdevice.h
MEMCPY = {"h2h": 0, "h2d": 1, "d2h": 2, "d2d": 3, "default": 4}
DTYPE = {"f32": 0, "bf16": 1, "f16": 2}
EXIT = {"none": 0, "relative": 1, "absolute": 2}


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = open(HEADER).read()
    return re.findall(r"^int\s+(pcd_\w+)\s*\(", text, flags=re.M)


def lib():
    """Load the library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(there is no fallback compute path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = c_int
        _lib = L
    return _lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(512)
    lib().pcd_last_error(buf, 512)
    return buf.value.decode(errors="replace")


def check(code: int, operation: str) -> None:
    """NativeCheck.Ok (Interop/CudaStatus.cs:31-37)."""
    if code != 0:
        raise DeviceException(code, operation, last_error())


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
