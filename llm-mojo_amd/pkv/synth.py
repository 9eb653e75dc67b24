"""Seeded N(0, 1) workload data generated on the device (libpkv_synth.so).

Value i of stream `seed` depends only on (seed, i) (a counter hash + Box-Muller, see
csrc/pkv_synth.hip), so the benchmark and the tests fill multi-GB pools in
milliseconds and download exactly the same values for the CPU reference when needed.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import hip

_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                     "libpkv_synth.so")
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_PATH):
            raise RuntimeError(f"{_PATH} not built: run `python llm-mojo_amd/build.py`")
        hip._lib()
        L = ctypes.CDLL(_PATH)
        L.pkv_synth_normal.restype = ctypes.c_int32
        L.pkv_synth_normal.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                       ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int32]
        _LIB = L
    return _LIB


def fill_normal(arr: hip.DeviceArray, seed: int, offset: int = 0, stream=None) -> hip.DeviceArray:
    """Fills a device array (float32, or uint16 holding bf16) with normal stream `seed`."""
    n = arr.nbytes // arr.dtype.itemsize
    dtype = 1 if arr.dtype == np.uint16 else 0
    if arr.dtype not in (np.float32, np.uint16):
        raise TypeError("fill_normal: float32 or uint16 (bf16) arrays only")
    rc = _lib().pkv_synth_normal(stream.handle if stream else None, arr.ptr, n, seed, offset,
                                 dtype)
    hip.check(rc, "pkv_synth_normal")
    return arr


def normal(shape, seed: int, dtype=np.float32, stream=None) -> hip.DeviceArray:
    return fill_normal(hip.DeviceArray(shape, dtype), seed, stream=stream)
