"""Minimal HIP runtime plumbing (device buffers, streams, events) over the same
libamdhip64 that libfirewing_hip_moe.so links, so callers and the library share
one runtime in the process. Used by the benchmark and the GPU tests to hand the
library device pointers and to time launches with HIP events on the launch
stream."""
from __future__ import annotations

import ctypes

import numpy as np

from . import hip_moe

_hip = None

H2D, D2H, D2D = 1, 2, 3


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        hip_moe.lib()  # loads /opt/rocm's libamdhip64 as the library's dependency
        L = ctypes.CDLL("libamdhip64.so.7")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        L.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        L.hipFree.argtypes = [vp]
        L.hipMemcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        L.hipMemset.argtypes = [vp, ctypes.c_int, sz]
        L.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        L.hipStreamDestroy.argtypes = [vp]
        L.hipStreamSynchronize.argtypes = [vp]
        L.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        L.hipEventDestroy.argtypes = [vp]
        L.hipEventRecord.argtypes = [vp, vp]
        L.hipEventSynchronize.argtypes = [vp]
        L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        L.hipGetErrorString.restype = ctypes.c_char_p
        L.hipGetErrorString.argtypes = [ctypes.c_int]
        _hip = L
    return _hip


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(status).decode()}")


class DeviceArray:
    """A device allocation holding a numpy-shaped array."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(hip().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, H2D), "hipMemcpy H2D")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def free(self) -> None:
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A default-priority HIP stream."""

    def __init__(self):
        s = ctypes.c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        check(hip().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            hip().hipStreamDestroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream) -> None:
        check(hip().hipEventRecord(self.handle, stream.handle), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(hip().hipEventSynchronize(end.handle), "hipEventSynchronize")
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle), "hipEventElapsedTime")
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            hip().hipEventDestroy(self.handle)
            self.handle = None
