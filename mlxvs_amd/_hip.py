"""Minimal HIP runtime access over ctypes: device buffers, copies, events.

Plumbing for callers that keep inputs resident in HBM (the benchmark, the
device-pointer tests).  The engine itself never imports this module.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.environ.get("MLXVS_HIP_RUNTIME", "libamdhip64.so")
        try:
            _LIB = ctypes.CDLL(path)
        except OSError:
            _LIB = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")
        _LIB.hipGetErrorString.restype = ctypes.c_char_p
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().hipGetErrorString(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} ({rc})")


def device_count() -> int:
    n = ctypes.c_int(0)
    rc = lib().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


class DeviceBuffer:
    """hipMalloc'ed memory, freed with the object."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        check(lib().hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(max(1, self.nbytes))),
              "hipMalloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().hipMemcpy(self.ptr, a.ctypes.data_as(ctypes.c_void_p),
                              ctypes.c_size_t(a.nbytes), 1), "hipMemcpy H2D")

    def download(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr,
                              ctypes.c_size_t(out.nbytes), 2), "hipMemcpy D2H")
        return out

    def free(self) -> None:
        if self.ptr:
            lib().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def value(self) -> int:
        return self.ptr.value or 0


def synchronize() -> None:
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Stream:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(lib().hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    def synchronize(self) -> None:
        check(lib().hipStreamSynchronize(self.handle), "hipStreamSynchronize")


class Event:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(lib().hipEventCreate(ctypes.byref(self.handle)), "hipEventCreate")

    def record(self, stream: Stream | None = None) -> None:
        s = stream.handle if stream is not None else ctypes.c_void_p()
        check(lib().hipEventRecord(self.handle, s), "hipEventRecord")

    def synchronize(self) -> None:
        check(lib().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        check(lib().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle),
              "hipEventElapsedTime")
        return ms.value
