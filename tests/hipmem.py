"""Device buffers for tests of the device-pointer entry points, through the HIP runtime the
product library itself loads (libamdhip64.so.7, the same instance by soname)."""
from __future__ import annotations

import ctypes as C

import numpy as np

import kurumi_amd as K

_H = None


def hip() -> C.CDLL:
    global _H
    if _H is None:
        K.lib()  # loads the runtime the product uses first
        L = C.CDLL("libamdhip64.so.7")
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipFree.argtypes = [C.c_void_p]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipDeviceSynchronize.argtypes = []
        L.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        L.hipStreamDestroy.argtypes = [C.c_void_p]
        L.hipStreamSynchronize.argtypes = [C.c_void_p]
        L.hipGetErrorString.restype = C.c_char_p
        _H = L
    return _H


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: HIP error {rc} ({hip().hipGetErrorString(rc).decode()})")


class DevBuf:
    """hipMalloc'd bytes, freed with the object."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        p = C.c_void_p()
        check(hip().hipMalloc(C.byref(p), max(nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @staticmethod
    def from_numpy(a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = DevBuf(a.nbytes)
        check(hip().hipMemcpy(b.ptr, a.ctypes.data, a.nbytes, 1), "hipMemcpy H2D")
        return b

    def numpy(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, 2), "hipMemcpy D2H")
        return out

    def __del__(self):
        if getattr(self, "ptr", None):
            hip().hipFree(self.ptr)
            self.ptr = None


def synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
