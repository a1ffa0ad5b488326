"""Minimal ctypes view of the HIP runtime that libkv-compact.so links.

Device buffers, copies, streams and events for tests and the benchmark,
bound to the same libamdhip64 instance as the library (dlopen by SONAME after
the library is loaded), so there is exactly one HIP runtime in the process.
"""
from __future__ import annotations

import ctypes

import numpy as np

H2D, D2H, D2D = 1, 2, 3

_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so.7")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        _hip.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        _hip.hipFree.argtypes = [vp]
        _hip.hipMemcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        _hip.hipMemcpyAsync.argtypes = [vp, vp, sz, ctypes.c_int, vp]
        _hip.hipMemset.argtypes = [vp, ctypes.c_int, sz]
        _hip.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        _hip.hipStreamSynchronize.argtypes = [vp]
        _hip.hipStreamDestroy.argtypes = [vp]
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        _hip.hipEventRecord.argtypes = [vp, vp]
        _hip.hipEventSynchronize.argtypes = [vp]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        _hip.hipEventDestroy.argtypes = [vp]
        _hip.hipDeviceGetName.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
        _hip.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        _hip.hipGetErrorString.restype = ctypes.c_char_p
        _hip.hipMemGetInfo.argtypes = [ctypes.POINTER(sz), ctypes.POINTER(sz)]
    return _hip


def check(rc, what="hip call"):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {hip().hipGetErrorString(rc).decode()} ({rc})")


class DevBuf:
    """Owned device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 1)), "hipMalloc")

    @property
    def value(self) -> int:
        return self.ptr.value

    def upload(self, arr: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes
        check(hip().hipMemcpy(self.ptr.value + offset, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(hip().hipMemcpy(out.ctypes.data, self.ptr.value + offset, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr.value:
            hip().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_count() -> int:
    n = ctypes.c_int(0)
    if hip().hipGetDeviceCount(ctypes.byref(n)) != 0:
        return 0
    return n.value


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    check(hip().hipDeviceGetName(buf, 256, 0), "hipDeviceGetName")
    return buf.value.decode()


def mem_free() -> int:
    """Free device memory in bytes (hipMemGetInfo)."""
    f, t = ctypes.c_size_t(0), ctypes.c_size_t(0)
    check(hip().hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)), "hipMemGetInfo")
    return f.value


def synchronize():
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Event:
    def __init__(self):
        self.e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(self.e)), "hipEventCreate")

    def record(self, stream=None):
        check(hip().hipEventRecord(self.e, stream), "hipEventRecord")

    def elapsed_ms(self, later: "Event") -> float:
        check(hip().hipEventSynchronize(later.e), "hipEventSynchronize")
        f = ctypes.c_float(0.0)
        check(hip().hipEventElapsedTime(ctypes.byref(f), self.e, later.e), "hipEventElapsedTime")
        return f.value
