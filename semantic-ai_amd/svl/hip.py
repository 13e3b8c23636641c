"""Minimal ctypes access to the HIP runtime that libsvl links (libamdhip64.so.7): device
buffers for the *_async entry points and events for timing on a state's stream."""
from __future__ import annotations

import ctypes as C

import numpy as np

_hip = None


def runtime():
    global _hip
    if _hip is None:
        h = C.CDLL("libamdhip64.so.7")
        vp = C.c_void_p
        h.hipMalloc.argtypes = [C.POINTER(vp), C.c_size_t]
        h.hipFree.argtypes = [vp]
        h.hipMemcpy.argtypes = [vp, vp, C.c_size_t, C.c_int]
        h.hipDeviceSynchronize.argtypes = []
        h.hipEventCreate.argtypes = [C.POINTER(vp)]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        h.hipEventDestroy.argtypes = [vp]
        h.hipGetErrorString.restype = C.c_char_p
        h.hipGetErrorString.argtypes = [C.c_int]
        _hip = h
    return _hip


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: {runtime().hipGetErrorString(rc).decode()}")


H2D, D2H = 1, 2


class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.ptr = C.c_void_p()
        self.nbytes = nbytes
        _ok(runtime().hipMalloc(C.byref(self.ptr), max(nbytes, 16)), "hipMalloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        _ok(runtime().hipMemcpy(buf.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes, H2D), "hipMemcpy")
        return buf

    def to_array(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _ok(runtime().hipMemcpy(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes, D2H), "hipMemcpy")
        return out

    @property
    def address(self) -> int:
        return self.ptr.value

    def free(self) -> None:
        if self.ptr:
            runtime().hipFree(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        self.free()


class Event:
    def __init__(self):
        self.e = C.c_void_p()
        _ok(runtime().hipEventCreate(C.byref(self.e)), "hipEventCreate")

    def record(self, stream: int) -> None:
        _ok(runtime().hipEventRecord(self.e, C.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, later: "Event") -> float:
        _ok(runtime().hipEventSynchronize(later.e), "hipEventSynchronize")
        ms = C.c_float()
        _ok(runtime().hipEventElapsedTime(C.byref(ms), self.e, later.e), "hipEventElapsedTime")
        return ms.value


def synchronize() -> None:
    _ok(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")
