"""ctypes prototypes of libpkv.so (declared in include/pkv.h).

The product path loads the in-tree library and fails loudly when it is missing:
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libpkv.so")

PKV_OK = 0
PKV_ERR_INVALID = -1
PKV_ERR_UNSUPPORTED = -2
PKV_ERR_WORKSPACE = -3
PKV_ERR_HIP = -4
PKV_DTYPE_F32 = 0
PKV_DTYPE_BF16 = 1
PKV_SEQ_OK = 0
PKV_SEQ_OUT_OF_BLOCKS = -1
PKV_SEQ_TABLE_FULL = -2
PKV_SEQ_BAD_BLOCK = -3
PKV_SEQ_FREE_OVERFLOW = -4
PKV_SEQ_BAD_ARGS = -5
PKV_SEQ_BAD_INDEX = -6

# Every exported entry point and its (restype, argtypes).
_vp, _i32, _sz, _f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t, ctypes.c_float


class PkvParams(ctypes.Structure):
    _fields_ = [
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("kv_dtype", ctypes.c_int32),
        ("ring_size", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_PP = ctypes.POINTER(PkvParams)
PROTOTYPES = {
    "pkv_workspace_size": (_sz, [_PP, _i32, _i32, _i32]),
    "pkv_append": (_i32, [_vp, _PP, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp,
                          _vp, _i32, _i32, _vp]),
    "pkv_attend": (_i32, [_vp, _PP, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp,
                          _sz]),
    "pkv_attend_noalloc": (_i32, [_vp, _PP, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32,
                                  _vp]),
    "pkv_decode": (_i32, [_vp, _PP, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _vp, _sz]),
    "pkv_rollback": (_i32, [_vp, _PP, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _vp]),
    "pkv_prefill": (_i32, [_vp, _PP, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _vp]),
    "pkv_paged_attention_layer": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                                         _i32, _vp, _i32, _i32, _i32, _i32, _vp, _sz]),
    "pkv_append_qkv": (_i32, [_vp, _PP, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp,
                              _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "pkv_sparse_workspace_size": (_sz, [_PP, _i32, _i32]),
    "pkv_attend_sparse": (_i32, [_vp, _PP, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _vp,
                                 _vp, _sz]),
    "pkv_verify": (_i32, [_vp, _PP, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _vp,
                          _vp, _sz]),
    "pkv_append_attend": (_i32, [_vp, _PP, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32,
                                 _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _sz]),
    "pkv_q4_matmul_workspace_size": (_sz, [_i32, _i32, _i32]),
    "pkv_q4_matmul": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _sz]),
    "pkv_lsa_max_keys": (_i32, [_i32, _i32, _i32]),
    "pkv_lsa_expand_workspace_size": (_sz, [_i32, _i32, _i32, _i32]),
    "pkv_lsa_expand": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp,
                              _i32, _i32, _vp, _vp, ctypes.c_int64, _vp, _vp, _sz]),
    "pkv_lsa_rollback": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "pkv_last_error": (ctypes.c_char_p, []),
    "pkv_version": (_i32, []),
}

_LIB = None


class PkvError(RuntimeError):
    def __init__(self, code: int, what: str, msg: str):
        super().__init__(f"{what} returned {code}: {msg}")
        self.code = code


def load(path: str | None = None) -> ctypes.CDLL:
    """Loads libpkv.so (in-tree) and declares its prototypes. Raises if it is missing."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(f"libpkv.so not built at {p}: run `python llm-mojo_amd/build.py` "
                           "(or __graft_entry__.build()) first")
    # Bind the HIP runtime first so libpkv resolves against the same instance.
    from . import hip as _hip  # noqa: F401
    _hip._lib()
    lib = ctypes.CDLL(p)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def call(name: str, *args) -> int:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != PKV_OK:
        raise PkvError(rc, name, lib.pkv_last_error().decode())
    return rc
