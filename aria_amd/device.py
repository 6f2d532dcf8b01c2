"""Device buffers, streams and events over the backend's C ABI (no torch).

``DeviceArray`` owns memory from aria_cuda_malloc and moves numpy arrays in and
out; ``Timer`` brackets stream work with HIP events. Used by bench.py and the
device-pointer tests.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import HipError, check, lib


class DeviceArray:
    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = lib().aria_cuda_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise HipError(f"aria_cuda_malloc({self.nbytes}) failed")

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            lib().aria_cuda_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes)
        return d

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            lib().aria_cuda_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes)
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes == self.nbytes
        lib().aria_cuda_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes)

    def free(self) -> None:
        if self.ptr:
            lib().aria_cuda_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def p(self):
        return self.ptr


def stream():
    return lib().aria_hip_default_stream()


def sync(s=None) -> None:
    check(lib().aria_hip_stream_sync(s), "stream sync")


class Timer:
    """HIP events on one stream: start() ... stop() -> milliseconds."""

    def __init__(self, s=None):
        self.s = s
        self.e0 = lib().aria_hip_event_create()
        self.e1 = lib().aria_hip_event_create()
        if not self.e0 or not self.e1:
            raise HipError("event create failed")

    def start(self) -> None:
        check(lib().aria_hip_event_record(self.e0, self.s), "event record")

    def stop(self) -> float:
        check(lib().aria_hip_event_record(self.e1, self.s), "event record")
        ms = lib().aria_hip_event_elapsed_ms(self.e0, self.e1)
        if ms < 0:
            raise HipError("event elapsed failed")
        return float(ms)

    def __del__(self):
        try:
            lib().aria_hip_event_destroy(self.e0)
            lib().aria_hip_event_destroy(self.e1)
        except Exception:
            pass


def cptr(p):
    return C.c_void_p(p)
