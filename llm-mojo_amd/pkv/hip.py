"""Minimal ctypes binding of the HIP runtime: device memory, copies, streams, events.

This is plumbing for the host side (tests, bench, the Python mirror of the engine's
host code); the product is libpkv.so. It binds the same libamdhip64 that libpkv.so
links, so both share one runtime instance.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HIP = None

hipMemcpyHostToDevice = 1
hipMemcpyDeviceToHost = 2
hipMemcpyDeviceToDevice = 3


class HipError(RuntimeError):
    pass


def _lib():
    global _HIP
    if _HIP is None:
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        path = os.path.join(rocm, "lib", "libamdhip64.so")
        _HIP = ctypes.CDLL(path)
        h = _HIP
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [i32]
        for name, args in {
            "hipMalloc": [ctypes.POINTER(vp), sz],
            "hipFree": [vp],
            "hipMemcpy": [vp, vp, sz, i32],
            "hipMemcpyAsync": [vp, vp, sz, i32, vp],
            "hipMemset": [vp, i32, sz],
            "hipMemsetAsync": [vp, i32, sz, vp],
            "hipDeviceSynchronize": [],
            "hipGetDeviceCount": [ctypes.POINTER(i32)],
            "hipSetDevice": [i32],
            "hipStreamCreate": [ctypes.POINTER(vp)],
            "hipStreamDestroy": [vp],
            "hipStreamSynchronize": [vp],
            "hipEventCreate": [ctypes.POINTER(vp)],
            "hipEventCreateWithFlags": [ctypes.POINTER(vp), ctypes.c_uint],
            "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipMemGetInfo": [ctypes.POINTER(sz), ctypes.POINTER(sz)],
        }.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = i32
    return _HIP


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib().hipGetErrorString(rc).decode()
        raise HipError(f"{what} failed: {msg} ({rc})")


def device_count() -> int:
    n = ctypes.c_int(0)
    rc = _lib().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


def synchronize() -> None:
    check(_lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info() -> tuple[int, int]:
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    check(_lib().hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
    return free.value, total.value


class DeviceArray:
    """A device allocation with a numpy dtype and shape (row-major)."""

    def __init__(self, shape, dtype, zero: bool = False):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(_lib().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value
        if zero:
            self.zero_()

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(arr.shape, arr.dtype)
        d.upload(arr)
        return d

    def upload(self, arr: np.ndarray, stream=None) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {arr.nbytes} vs {self.nbytes}")
        check(_lib().hipMemcpy(self.ptr, arr.ctypes.data, self.nbytes, hipMemcpyHostToDevice),
              "hipMemcpy H2D")

    def upload_at(self, byte_offset: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if byte_offset < 0 or byte_offset + arr.nbytes > self.nbytes:
            raise ValueError("upload_at out of range")
        check(_lib().hipMemcpy(self.ptr + byte_offset, arr.ctypes.data, arr.nbytes,
                               hipMemcpyHostToDevice), "hipMemcpy H2D")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(_lib().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, hipMemcpyDeviceToHost),
              "hipMemcpy D2H")
        return out

    def zero_(self) -> None:
        check(_lib().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def fill_bytes_(self, value: int) -> None:
        check(_lib().hipMemset(self.ptr, value, self.nbytes), "hipMemset")

    def copy_from(self, other: "DeviceArray") -> None:
        if other.nbytes != self.nbytes:
            raise ValueError("size mismatch")
        check(_lib().hipMemcpy(self.ptr, other.ptr, self.nbytes, hipMemcpyDeviceToDevice),
              "hipMemcpy D2D")

    def free(self) -> None:
        if getattr(self, "ptr", None):
            _lib().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(_lib().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        check(_lib().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            _lib().hipStreamDestroy(self.handle)
            self.handle = None


hipEventDisableSystemFence = 0x20000000  # record without a system-scope release


class Event:
    def __init__(self, flags: int = 0):
        e = ctypes.c_void_p()
        if flags:
            check(_lib().hipEventCreateWithFlags(ctypes.byref(e), flags),
                  "hipEventCreateWithFlags")
        else:
            check(_lib().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream | None = None) -> None:
        check(_lib().hipEventRecord(self.handle, stream.handle if stream else None),
              "hipEventRecord")

    def synchronize(self) -> None:
        check(_lib().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(_lib().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle),
              "hipEventElapsedTime")
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            _lib().hipEventDestroy(self.handle)
            self.handle = None
