"""Minimal ctypes access to the HIP runtime (device buffers, copies, streams, events) for the
benchmark and device-pointer tests. Plumbing only; all compute lives in libllmembed_hip.so."""
from __future__ import annotations

import ctypes as C
import glob
import os

import numpy as np

_RT = None


def rt():
    global _RT
    if _RT is None:
        cands = [os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so")]
        cands += sorted(glob.glob("/opt/rocm*/lib/libamdhip64.so*"))
        last = None
        for c in cands:
            try:
                _RT = C.CDLL(c)
                break
            except OSError as e:  # pragma: no cover
                last = e
        if _RT is None:
            raise RuntimeError(f"libamdhip64.so not found: {last}")
        P = C.c_void_p
        _RT.hipMalloc.argtypes = [C.POINTER(P), C.c_size_t]
        _RT.hipFree.argtypes = [P]
        _RT.hipMemcpy.argtypes = [P, P, C.c_size_t, C.c_int]
        _RT.hipMemset.argtypes = [P, C.c_int, C.c_size_t]
        _RT.hipDeviceSynchronize.argtypes = []
        _RT.hipStreamCreate.argtypes = [C.POINTER(P)]
        _RT.hipStreamSynchronize.argtypes = [P]
        _RT.hipEventCreate.argtypes = [C.POINTER(P)]
        _RT.hipEventRecord.argtypes = [P, P]
        _RT.hipEventSynchronize.argtypes = [P]
        _RT.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), P, P]
        _RT.hipSetDevice.argtypes = [C.c_int]
    return _RT


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError {rc}")


H2D, D2H, D2D = 1, 2, 3


class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.ptr = C.c_void_p()
        _ok(rt().hipMalloc(C.byref(self.ptr), max(int(nbytes), 256)), "hipMalloc")
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        _ok(rt().hipMemcpy(self.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        _ok(rt().hipMemcpy(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    @property
    def value(self) -> int:
        return self.ptr.value

    def free(self):
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    _ok(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Stream:
    def __init__(self):
        self.h = C.c_void_p()
        _ok(rt().hipStreamCreate(C.byref(self.h)), "hipStreamCreate")

    def synchronize(self):
        _ok(rt().hipStreamSynchronize(self.h), "hipStreamSynchronize")


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        _ok(rt().hipEventCreate(C.byref(self.h)), "hipEventCreate")

    def record(self, stream: Stream | None = None):
        _ok(rt().hipEventRecord(self.h, stream.h if stream else None), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        _ok(rt().hipEventSynchronize(end.h), "hipEventSynchronize")
        ms = C.c_float()
        _ok(rt().hipEventElapsedTime(C.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value
