"""Loads liblokinfer_hip.so (the gfx950 kernels + registry C-ABI, include/lokinfer_hip.h) with ctypes.

The library is the only compute path: if it is missing this module raises, it never falls back to anything.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liblokinfer_hip.so"

_lib = None


class LokinferError(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("LOKINFER_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise LokinferError(f"{path} is not built: run `python -m lokinfer_amd.build` (hipcc, gfx950)")
    L = C.CDLL(str(path))
    vp, i64, u32, i32 = C.c_void_p, C.c_int64, C.c_uint32, C.c_int
    L.lk_init.restype = i32
    L.lk_num_kernels.restype = i32
    L.lk_kernel_name_at.argtypes = [i32]
    L.lk_kernel_name_at.restype = C.c_char_p
    L.lk_find_kernel.argtypes = [C.c_char_p]
    L.lk_find_kernel.restype = vp
    L.lk_kernel_is_gpu.argtypes = [vp]
    L.lk_kernel_is_gpu.restype = i32
    L.lk_kernel_arity.argtypes = [vp, C.POINTER(i32), C.POINTER(i32)]
    L.lk_kernel_arity.restype = i32
    L.lk_run_kernel.argtypes = [vp, C.POINTER(vp), u32, C.POINTER(i64), u32, C.POINTER(C.c_double), u32, vp,
                                C.c_uint64, vp]
    L.lk_run_kernel.restype = i32
    L.lk_last_error.restype = C.c_char_p
    L.lk_take_device_error.argtypes = [C.POINTER(i64)]
    L.lk_take_device_error.restype = i32
    L.lk_device_error_message.argtypes = [i32]
    L.lk_device_error_message.restype = C.c_char_p
    L.lk_init()
    _lib = L
    return L


def check_device_errors() -> None:
    """Waits for the current GPU and raises LokinferError if a kernel recorded a data error since the last check
    (a position outside a KV cache, an id out of range, a persistent kernel whose exchange timed out); clears it.
    The reference reports GPU failures the same way, at its next synchronisation (takeGpuError,
    src/runtime/executable.cpp:850-852 in lariaus/lokinfer)."""
    L = lib()
    detail = C.c_int64(0)
    code = L.lk_take_device_error(C.byref(detail))
    if code < 0:
        raise LokinferError("could not read the device error record")
    if code:
        raise LokinferError(f"device error {code}: {L.lk_device_error_message(code).decode()} (detail {detail.value})")


def registered_kernels() -> list[str]:
    L = lib()
    return [L.lk_kernel_name_at(i).decode() for i in range(L.lk_num_kernels())]


def exported_symbols() -> set[str]:
    """Names of the C-ABI functions include/lokinfer_hip.h declares that the library exports."""
    import re

    hdr = Path(__file__).resolve().parent.parent / "include" / "lokinfer_hip.h"
    names = set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(lk_\w+)\s*\(", hdr.read_text(), re.M))
    L = lib()
    return {n for n in names if hasattr(L, n)}
