"""Device memory, streams and events through the C ABI (no torch).

The GPU path of this package never imports torch: torch ships its own HIP
runtime, and a second runtime in the process would be a hazard. Buffers here
are plain device allocations made by libkvflux_hip.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import capi


class DeviceBuffer:
    """Owning device allocation of `nbytes` on the current device."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        capi.call("kvflux_device_malloc", C.byref(p), max(self.nbytes, 1))
        self.ptr = int(p.value)

    def free(self) -> None:
        if self.ptr:
            capi.call("kvflux_device_free", C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, array: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(array)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload exceeds buffer")
        capi.call("kvflux_memcpy", C.c_void_p(self.ptr + offset), C.c_void_p(a.ctypes.data), a.nbytes)

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dt)
        if out.nbytes:
            capi.call("kvflux_memcpy", C.c_void_p(out.ctypes.data), C.c_void_p(self.ptr + offset),
                      out.nbytes)
        return out

    def fill(self, byte: int, stream: int = 0) -> None:
        capi.call("kvflux_fill_bytes", C.c_void_p(self.ptr), int(byte), self.nbytes, C.c_void_p(stream))
        synchronize(stream)


def to_device(array: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(array)
    buf = DeviceBuffer(a.nbytes)
    buf.upload(a)
    return buf


def synchronize(stream: int = 0) -> None:
    capi.call("kvflux_stream_synchronize", C.c_void_p(stream))


def memcpy_d2h(ptr: int, nbytes: int, dtype) -> np.ndarray:
    dt = np.dtype(dtype)
    out = np.empty(nbytes // dt.itemsize, dtype=dt)
    if nbytes:
        capi.call("kvflux_memcpy", C.c_void_p(out.ctypes.data), C.c_void_p(ptr), nbytes)
    return out


def memcpy_h2d(ptr: int, array: np.ndarray) -> None:
    a = np.ascontiguousarray(array)
    if a.nbytes:
        capi.call("kvflux_memcpy", C.c_void_p(ptr), C.c_void_p(a.ctypes.data), a.nbytes)


def fill_random(ptr: int, count: int, dtype: int, distribution: int, seed: int, stream: int = 0) -> None:
    capi.call("kvflux_fill_random", C.c_void_p(ptr), int(count), int(dtype), int(distribution),
              int(seed) & (2**64 - 1), C.c_void_p(stream))


def compare_bytes(a: int, b: int, nbytes: int) -> int:
    out = C.c_uint64(0)
    capi.call("kvflux_compare_bytes", C.c_void_p(a), C.c_void_p(b), int(nbytes), C.byref(out))
    return int(out.value)


class Stream:
    def __init__(self):
        s = C.c_void_p()
        capi.call("kvflux_stream_create", C.byref(s))
        self.handle = int(s.value or 0)

    def synchronize(self) -> None:
        synchronize(self.handle)

    def __del__(self):
        try:
            if self.handle:
                capi.call("kvflux_stream_destroy", C.c_void_p(self.handle))
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        capi.call("kvflux_event_create", C.byref(e))
        self.handle = int(e.value)

    def record(self, stream: int = 0) -> None:
        capi.call("kvflux_event_record", C.c_void_p(self.handle), C.c_void_p(stream))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        capi.call("kvflux_event_elapsed_ms", C.byref(ms), C.c_void_p(self.handle), C.c_void_p(end.handle))
        return float(ms.value)

    def __del__(self):
        try:
            capi.call("kvflux_event_destroy", C.c_void_p(self.handle))
        except Exception:
            pass
