"""Minimal ctypes access to the HIP runtime that libvxs.so itself is linked against: device buffers,
copies and events for device-resident calls and kernel timing, without a second HIP runtime in the
process.

torch wheels bundle their own libamdhip64; a process that uses torch tensors with this library must
import torch *before* voxwerk_amd so that libvxs binds to torch's copy (same soname).
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_size_t, c_void_p

import numpy as np

from ._lib import load_vxs

_hip = None

H2D, D2H, D2D = 1, 2, 3


def lib() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        load_vxs()  # resolves libamdhip64.so.7 first; this returns the already-loaded instance
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [ctypes.POINTER(c_void_p), c_size_t]
        h.hipFree.argtypes = [c_void_p]
        h.hipMemcpy.argtypes = [c_void_p, c_void_p, c_size_t, c_int]
        h.hipMemcpyAsync.argtypes = [c_void_p, c_void_p, c_size_t, c_int, c_void_p]
        h.hipMemset.argtypes = [c_void_p, c_int, c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamSynchronize.argtypes = [c_void_p]
        h.hipEventCreate.argtypes = [ctypes.POINTER(c_void_p)]
        h.hipEventDestroy.argtypes = [c_void_p]
        h.hipEventRecord.argtypes = [c_void_p, c_void_p]
        h.hipEventSynchronize.argtypes = [c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(c_float), c_void_p, c_void_p]
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [c_int]
        _hip = h
    return _hip


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: {lib().hipGetErrorString(rc).decode()} ({rc})")


class DeviceArray:
    """A device allocation with numpy-style shape/dtype bookkeeping."""

    def __init__(self, shape, dtype):
        self.shape = tuple(np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = c_void_p()
        check(lib().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes == self.nbytes
        check(lib().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, H2D), "hipMemcpy H2D")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(lib().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, other: "DeviceArray") -> None:
        assert other.nbytes == self.nbytes
        check(lib().hipMemcpy(self.ptr, other.ptr, self.nbytes, D2D), "hipMemcpy D2D")

    def data_ptr(self) -> int:
        return self.ptr

    def free(self) -> None:
        if self.ptr:
            lib().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = c_void_p()
        check(lib().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.h = e.value

    def record(self, stream: int | None) -> None:
        check(lib().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(lib().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        check(lib().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            lib().hipEventDestroy(self.h)
        except Exception:
            pass


def synchronize() -> None:
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def stream_synchronize(stream: int | None) -> None:
    check(lib().hipStreamSynchronize(stream), "hipStreamSynchronize")
