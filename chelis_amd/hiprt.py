"""Minimal ctypes access to the HIP runtime for timing and synchronization
(events recorded on the library's own stream). Plumbing only."""
from __future__ import annotations

import ctypes
import os

_hip = None


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        for cand in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                _hip = ctypes.CDLL(cand)
                break
            except OSError:
                continue
        if _hip is None:
            raise RuntimeError("libamdhip64.so not found")
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        _hip.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        _hip.hipDeviceGetName = getattr(_hip, "hipDeviceGetName", None)
    return _hip


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed: hipError {rc}")


def device_count() -> int:
    n = ctypes.c_int(0)
    rc = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


class Event:
    def __init__(self):
        self.h = ctypes.c_void_p()
        _ok(hip().hipEventCreate(ctypes.byref(self.h)), "hipEventCreate")

    def record(self, stream):
        _ok(hip().hipEventRecord(self.h, ctypes.c_void_p(stream)), "hipEventRecord")

    def synchronize(self):
        _ok(hip().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _ok(hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            hip().hipEventDestroy(self.h)
        except Exception:
            pass


def device_synchronize():
    _ok(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
