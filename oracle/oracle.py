"""numpy bindings of the CPU oracle (oracle/pkv_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module. Function
docstrings name the reference code each restates (phildrip/llm-mojo, file:line).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
# PKV_ORACLE_LIB selects another build of the same source (the sanitizer build of
# `make -C oracle sanitize`, or the AVX-512 build the benchmark times).
LIB_PATH = os.environ.get("PKV_ORACLE_LIB") or os.path.join(ORACLE_DIR, "libpkv_oracle.so")
LIB_V4_PATH = os.path.join(ORACLE_DIR, "libpkv_oracle_v4.so")

F32, BF16 = 0, 1
_lib = None


def host_has_avx512() -> bool:
    """True when this host's CPU runs x86-64-v4 code (AVX-512 F, BW, CD, DQ, VL)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags
    except OSError:
        pass
    return False


def use_host_build() -> str:
    """Loads the build for this host's ISA level (the AVX-512 one where the CPU has it and
    it is built) before the first oracle call; returns the path in use. The builds differ
    only in vector width: every restated loop keeps its own summation order."""
    global LIB_PATH
    if _lib is None and "PKV_ORACLE_LIB" not in os.environ and host_has_avx512() \
            and os.path.exists(LIB_V4_PATH):
        LIB_PATH = LIB_V4_PATH
    return LIB_PATH


def _L():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: run `make -C {ORACLE_DIR}`")
        L = ctypes.CDLL(LIB_PATH)
        i64, i32, vp, f32 = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_float
        sig = {
            "pkvo_window_start": (i64, [i64, i64]),
            "pkvo_ring_row": (i64, [i64, i64, i64]),
            "pkvo_paged_attention_layer": (ctypes.c_int, [vp, vp, vp, ctypes.c_int, vp, i64, i64,
                                                          i64, i64, i64, i64, i64, vp, vp, vp,
                                                          i64, i64, ctypes.c_int]),
            "pkvo_legacy_paged_attention": (None, [vp, vp, vp, ctypes.c_int, vp, i64, i64, i64,
                                                   i64, i64, vp, vp]),
            "pkvo_attention_f64": (None, [vp, vp, vp, ctypes.c_int, vp, i64, i64, i64, i64, i64,
                                          i64, vp]),
            "pkvo_lcg_init": (ctypes.c_uint64, [ctypes.c_uint64]),
            "pkvo_fill_random": (ctypes.c_uint64, [vp, i64, f32, ctypes.c_uint64]),
            "pkvo_f32_to_bf16_array": (None, [vp, vp, i64]),
            "pkvo_bm_init": (None, [vp, vp, i32]),
            "pkvo_bm_allocate": (i32, [vp, vp]),
            "pkvo_bm_free": (None, [vp, vp, i32]),
            "pkvo_append": (None, [ctypes.c_int, i32, i32, vp, vp, vp, i32, vp, vp, vp, vp, vp,
                                   i32, vp, vp, i32, i32, vp]),
            "pkvo_ring_append": (None, [ctypes.c_int, i32, i32, i32, vp, vp, vp, i32, vp, vp, i32,
                                        vp, vp, i32, i32, vp]),
            "pkvo_rollback": (None, [i32, vp, i32, vp, vp, vp, vp, i32]),
            "pkvo_attend": (ctypes.c_int, [ctypes.c_int, i32, i32, i32, i32, i32, f32, vp, vp, vp,
                                           vp, i32, vp, vp, i32, i32, vp, ctypes.c_int,
                                           ctypes.c_int, i32]),
            "pkvo_attend_f64": (ctypes.c_int, [ctypes.c_int, i32, i32, i32, i32, i32, f32, vp,
                                               vp, vp, vp, i32, vp, i32, i32, vp, ctypes.c_int,
                                               i32]),
            "pkvo_max_threads": (ctypes.c_int, []),
            "pkvo_rms_norm": (None, [vp, vp, vp, i64]),
            "pkvo_rms_norm_noscale": (None, [vp, vp, i64]),
            "pkvo_apply_rope": (None, [vp, i64, i64, i64, ctypes.c_int]),
            "pkvo_apply_rope_qk": (None, [vp, vp, i64, i64, i64, i64, ctypes.c_int]),
            "pkvo_ref_apply_rope": (None, [vp, i64, i64, i64, ctypes.c_int]),
            "pkvo_lsa_sparse_paged_attention": (None, [vp, vp, vp, ctypes.c_int, vp, i64, vp, i64,
                                                       i64, i64, i64, vp, vp, vp, ctypes.c_int]),
            "pkvo_lsa_expand_buckets": (i64, [vp, i64, vp, vp, i64, i64, i64, i64, i64, vp]),
            "pkvo_lsa_reset": (None, [i64, vp, vp, vp]),
            "pkvo_lsa_rollback_to": (None, [i64, i64, vp, vp, vp, i64]),
            "pkvo_attend_sparse": (None, [ctypes.c_int, i32, i32, i32, i32, f32, vp, vp, vp, vp,
                                          i32, vp, vp, i32, vp, ctypes.c_int, ctypes.c_int]),
            "pkvo_attend_sparse_f64": (None, [ctypes.c_int, i32, i32, i32, i32, f32, vp, vp, vp,
                                              vp, i32, vp, vp, i32, vp]),
            "pkvo_quantize_q4_0": (None, [vp, vp, vp, i64]),
            "pkvo_q4_matmul_vec": (None, [vp, vp, vp, vp, i64, i64]),
            "pkvo_scalar_q4": (None, [vp, vp, vp, vp, i64, i64]),
            "pkvo_q4_matmul_f64": (None, [vp, vp, vp, vp, i64, i64]),
            "pkvo_append_qkv_f64": (None, [i32, i32, i32, ctypes.c_int, vp, vp, i32, vp, vp, vp,
                                           vp, vp, i32, i32, vp, vp, vp]),
            "pkvo_append_qkv": (None, [ctypes.c_int, i32, i32, i32, i32, i32, i32, ctypes.c_int,
                                       vp, vp, vp, i32, vp, vp, vp, vp, vp, i32, vp, vp, vp, vp,
                                       vp, vp, i32, i32, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _dtype_of(pool: np.ndarray) -> int:
    if pool.dtype == np.float32:
        return F32
    if pool.dtype == np.uint16:
        return BF16
    raise TypeError(f"pool dtype {pool.dtype} (want float32 or uint16 bf16 bits)")


def max_threads() -> int:
    return _L().pkvo_max_threads()


def window_start(pos: int, window: int) -> int:
    """attention.mojo:135-141"""
    return _L().pkvo_window_start(pos, window)


def ring_row(slot: int, ring_size: int, t: int) -> int:
    """attention.mojo:144-148"""
    return _L().pkvo_ring_row(slot, ring_size, t)


def paged_attention_layer(q, k_pool, v_pool, block_table, block_size, pos, num_heads,
                          num_kv_heads, head_dim, window, scores=None, rows=None, attn_out=None,
                          ring_size=0, ring_base=0, nthreads=1):
    """3-pass fp32 attention, attention.mojo:240-294 (+ :151-237). Returns attn_out.
    scores / rows may be given to check the scratch contract (scores >= Hq*n, rows >= n)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    tab = np.ascontiguousarray(np.asarray(block_table, dtype=np.int64))
    n = pos + 1 - window_start(pos, window)
    if scores is None:
        scores = np.empty(max(num_heads * n, 1), np.float32)
    if rows is None:
        rows = np.empty(max(n, 1), np.int64)
    if attn_out is None:
        attn_out = np.empty(num_heads * head_dim, np.float32)
    rc = _L().pkvo_paged_attention_layer(_p(q), _p(k_pool), _p(v_pool), _dtype_of(k_pool),
                                         _p(tab), tab.size, block_size, pos, num_heads,
                                         num_kv_heads, head_dim, window, _p(scores), _p(rows),
                                         _p(attn_out), ring_size, ring_base, nthreads)
    if rc != 0:
        raise RuntimeError(f"paged_attention_layer rc={rc}")
    return attn_out


def legacy_paged_attention(q, k_pool, v_pool, block_table, block_size, pos, heads, kv_heads,
                           head_dim):
    """test_attention.mojo:62-117 (the engine's pre-refactor loop)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    tab = np.ascontiguousarray(np.asarray(block_table, dtype=np.int64))
    scores = np.empty(pos + 1, np.float32)
    out = np.empty(heads * head_dim, np.float32)
    _L().pkvo_legacy_paged_attention(_p(q), _p(k_pool), _p(v_pool), _dtype_of(k_pool), _p(tab),
                                     block_size, pos, heads, kv_heads, head_dim, _p(scores),
                                     _p(out))
    return out


def attention_f64(q, k_pool, v_pool, block_table, block_size, pos, start_t, heads, kv_heads,
                  head_dim):
    """test_attention.mojo:123-163 (naive float64 reference)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    tab = np.ascontiguousarray(np.asarray(block_table, dtype=np.int64))
    out = np.empty(heads * head_dim, np.float64)
    _L().pkvo_attention_f64(_p(q), _p(k_pool), _p(v_pool), _dtype_of(k_pool), _p(tab),
                            block_size, pos, start_t, heads, kv_heads, head_dim, _p(out))
    return out


def rms_norm(x, w) -> np.ndarray:
    """…batched.mojo:857-867 (one head: len(x) % 8 == 0)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    _L().pkvo_rms_norm(_p(x), _p(w), _p(out), x.size)
    return out


def rms_norm_noscale(x) -> np.ndarray:
    """…batched.mojo:870-878."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _L().pkvo_rms_norm_noscale(_p(x), _p(out), x.size)
    return out


def apply_rope(vec, num_heads, head_dim, pos, is_global) -> np.ndarray:
    """attention.mojo:24-66 (returns a rotated copy)."""
    v = np.array(vec, np.float32, copy=True).reshape(-1)
    _L().pkvo_apply_rope(_p(v), num_heads, head_dim, pos, int(is_global))
    return v


def apply_rope_qk(q, k, num_q_heads, num_kv_heads, head_dim, pos, is_global):
    """attention.mojo:69-132 (returns rotated copies)."""
    q = np.array(q, np.float32, copy=True).reshape(-1)
    k = np.array(k, np.float32, copy=True).reshape(-1)
    _L().pkvo_apply_rope_qk(_p(q), _p(k), num_q_heads, num_kv_heads, head_dim, pos,
                            int(is_global))
    return q, k


def ref_apply_rope(vec, num_heads, head_dim, pos, is_global) -> np.ndarray:
    """test_rope_and_parallel_attn.mojo:9-29 (scalar per-element RoPE)."""
    v = np.array(vec, np.float32, copy=True).reshape(-1)
    _L().pkvo_ref_apply_rope(_p(v), num_heads, head_dim, pos, int(is_global))
    return v


def append_qkv(state, layer, pos, tok_off, q, k, v, q_norm_w, k_norm_w, max_new, num_heads,
               num_kv_heads, head_dim, is_global, slots=None):
    """pkvo_append_qkv on a CacheState (paged) or RingState (ring; `slots` = ring slot of
    each sequence). Returns (status, q_out); q_out rows of skipped sequences are NaN."""
    pos = np.ascontiguousarray(pos, np.int32)
    tok_off = np.ascontiguousarray(tok_off, np.int32)
    q = np.ascontiguousarray(q, np.float32).reshape(-1, num_heads * head_dim)
    k = np.ascontiguousarray(k, np.float32).reshape(-1, num_kv_heads * head_dim)
    vv = None if v is None else np.ascontiguousarray(v, np.float32).reshape(k.shape)
    qw = np.ascontiguousarray(q_norm_w, np.float32)
    kw = np.ascontiguousarray(k_norm_w, np.float32)
    batch = pos.size
    status = np.zeros(batch, np.int32)
    q_out = np.full(q.shape, np.nan, np.float32)
    dt = BF16 if state.dtype == np.uint16 else F32
    ring = isinstance(state, RingState)
    if ring:
        tables = np.ascontiguousarray(slots, np.int32)
        args = (0, state.ring_size, state.num_slots, _p(tables), 1, None, None, None)
    else:
        args = (state.block_size, 0, state.num_blocks, _p(state.tables), state.table_stride,
                _p(state.table_lens), _p(state.bm.free_list), _p(state.bm.count))
    bs, ring_size, nblk, tab, stride, lens, fl, fc = args
    _L().pkvo_append_qkv(dt, num_heads, num_kv_heads, head_dim, bs, ring_size, nblk,
                         int(is_global), _p(state.k_pools[layer]), _p(state.v_pools[layer]), tab,
                         stride, lens, fl, fc, _p(pos), _p(tok_off), max_new, _p(q), _p(k),
                         None if vv is None else _p(vv), _p(qw), _p(kw), _p(q_out), q.shape[0],
                         batch, _p(status))
    return status, q_out


def producer_f64(pos, tok_off, q, k, v, q_norm_w, k_norm_w, max_new, num_heads, num_kv_heads,
                 head_dim, is_global):
    """Exact (float64) processed rows of append_qkv's producer step, in input row layout:
    (q, k, v) float64 arrays; rows of sequences without a usable token range are NaN."""
    pos = np.ascontiguousarray(pos, np.int32)
    tok_off = np.ascontiguousarray(tok_off, np.int32)
    q = np.ascontiguousarray(q, np.float32).reshape(-1, num_heads * head_dim)
    k = np.ascontiguousarray(k, np.float32).reshape(-1, num_kv_heads * head_dim)
    vv = None if v is None else np.ascontiguousarray(v, np.float32).reshape(k.shape)
    qw = np.ascontiguousarray(q_norm_w, np.float32)
    kw = np.ascontiguousarray(k_norm_w, np.float32)
    qo = np.full(q.shape, np.nan)
    ko = np.full(k.shape, np.nan)
    vo = np.full(k.shape, np.nan)
    _L().pkvo_append_qkv_f64(num_heads, num_kv_heads, head_dim, int(is_global), _p(pos),
                             _p(tok_off), max_new, _p(q), _p(k), None if vv is None else _p(vv),
                             _p(qw), _p(kw), q.shape[0], pos.size, _p(qo), _p(ko), _p(vo))
    return qo, ko, vo


def lsa_sparse_paged_attention(q, k_pool, v_pool, block_table, block_size, selected, num_heads,
                               num_kv_heads, head_dim, nthreads=1):
    """lsa_core.mojo:630-680 (single query, explicit key list). Returns attn_out."""
    q = np.ascontiguousarray(q, np.float32)
    tab = np.ascontiguousarray(np.asarray(block_table, dtype=np.int64))
    sel = np.ascontiguousarray(np.asarray(selected, dtype=np.int64))
    n = max(sel.size, 1)
    scores = np.empty(num_heads * n, np.float32)
    rows = np.empty(n, np.int64)
    out = np.empty(num_heads * head_dim, np.float32)
    _L().pkvo_lsa_sparse_paged_attention(_p(q), _p(k_pool), _p(v_pool), _dtype_of(k_pool),
                                         _p(tab), block_size, _p(sel), sel.size, num_heads,
                                         num_kv_heads, head_dim, _p(scores), _p(rows), _p(out),
                                         nthreads)
    return out


def lsa_expand_buckets(picked, sizes, members, pos, top_k, sink_size, window_size):
    """lsa_core.mojo:573-604. members: [buckets][bucket_cap]. Returns the key list."""
    picked = np.ascontiguousarray(np.asarray(picked, dtype=np.int64))
    sizes = np.ascontiguousarray(np.asarray(sizes, dtype=np.int64))
    members = np.ascontiguousarray(np.asarray(members, dtype=np.int64))
    out = np.empty(max(top_k, 1) + max(window_size, 0) + max(sink_size, 0), np.int64)
    n = _L().pkvo_lsa_expand_buckets(_p(picked), picked.size, _p(sizes), _p(members),
                                     members.shape[1], pos, top_k, sink_size, window_size, _p(out))
    return out[:n].copy()


class LsaIndexState:
    """The integer state of one LSALayerIndex (lsa_core.mojo:222-233, :246-262): closed
    cluster blocks, tokens appended, and per-bucket member counts."""

    def __init__(self, max_capacity: int):
        self.max_capacity = max_capacity
        self.max_buckets = (max_capacity + 511) // 512 * 32
        self.closed_blocks = np.zeros(1, np.int64)
        self.total_tokens = np.zeros(1, np.int64)
        self.sizes = np.zeros(self.max_buckets, np.int64)

    def reset(self):
        """lsa_core.mojo:281-285."""
        _L().pkvo_lsa_reset(self.max_buckets, _p(self.closed_blocks), _p(self.total_tokens),
                            _p(self.sizes))

    def rollback_to(self, target_tokens: int):
        """lsa_core.mojo:287-303."""
        _L().pkvo_lsa_rollback_to(self.max_capacity, self.max_buckets, _p(self.closed_blocks),
                                  _p(self.total_tokens), _p(self.sizes), target_tokens)


def attend_sparse(q, k_pool, v_pool, tables, keys, key_off, num_heads, num_kv_heads, head_dim,
                  block_size, scale=1.0, nthreads=1, par=0):
    """One lsa_sparse_paged_attention call per sequence; q: [batch, Hq, D] fp32."""
    q = np.ascontiguousarray(q, np.float32)
    tables = np.ascontiguousarray(tables, np.int32)
    keys = np.ascontiguousarray(keys, np.int32)
    key_off = np.ascontiguousarray(key_off, np.int32)
    batch = key_off.size - 1
    out = np.empty((batch, num_heads, head_dim), np.float32)
    _L().pkvo_attend_sparse(_dtype_of(k_pool), num_heads, num_kv_heads, head_dim, block_size,
                            scale, _p(q), _p(k_pool), _p(v_pool), _p(tables), tables.shape[1],
                            _p(keys), _p(key_off), batch, _p(out), nthreads, par)
    return out


def attend_sparse_f64(q, k_pool, v_pool, tables, keys, key_off, num_heads, num_kv_heads,
                      head_dim, block_size, scale=1.0):
    """Exact (float64) attention over each sequence's key list."""
    q = np.ascontiguousarray(q, np.float32)
    tables = np.ascontiguousarray(tables, np.int32)
    keys = np.ascontiguousarray(keys, np.int32)
    key_off = np.ascontiguousarray(key_off, np.int32)
    batch = key_off.size - 1
    out = np.empty((batch, num_heads, head_dim), np.float64)
    _L().pkvo_attend_sparse_f64(_dtype_of(k_pool), num_heads, num_kv_heads, head_dim, block_size,
                                scale, _p(q), _p(k_pool), _p(v_pool), _p(tables), tables.shape[1],
                                _p(keys), _p(key_off), batch, _p(out))
    return out


def quantize_q4_0(w) -> tuple[np.ndarray, np.ndarray]:
    """moe_kernels.mojo:7-57 on a [rows][c_in] fp32 matrix: (packed uint8 [rows][c_in/2],
    scales fp32 [rows][c_in/32])."""
    w = np.ascontiguousarray(w, np.float32)
    rows, c_in = w.shape
    packed = np.empty((rows, c_in // 2), np.uint8)
    scales = np.empty((rows, c_in // 32), np.float32)
    _L().pkvo_quantize_q4_0(_p(w), _p(packed), _p(scales), w.size)
    return packed, scales


def q4_matmul_vec(packed, scales, x) -> np.ndarray:
    """moe_kernels.mojo:59-163: out[r] for one input vector x [c_in]."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(packed.shape[0], np.float32)
    _L().pkvo_q4_matmul_vec(_p(packed), _p(scales), _p(x), _p(out), x.size, packed.shape[0])
    return out


def scalar_q4(packed, scales, x) -> np.ndarray:
    """test_q4_4row_tiling.mojo:14-34 (independent scalar oracle)."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(packed.shape[0], np.float32)
    _L().pkvo_scalar_q4(_p(packed), _p(scales), _p(x), _p(out), x.size, packed.shape[0])
    return out


def q4_matmul_f64(packed, scales, x) -> np.ndarray:
    """The dequantized product in float64."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(packed.shape[0], np.float64)
    _L().pkvo_q4_matmul_f64(_p(packed), _p(scales), _p(x), _p(out), x.size, packed.shape[0])
    return out


class Lcg:
    """test_attention.mojo:27-37 -- uniform [-1, 1) from a 64-bit LCG."""

    def __init__(self, seed: int):
        self.state = _L().pkvo_lcg_init(seed)

    def fill(self, n: int, scale: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.state = _L().pkvo_fill_random(_p(out), n, scale, self.state)
        return out


def shuffled_block_table(num_logical: int, num_blocks: int) -> np.ndarray:
    """test_attention.mojo:45-50 -- (i*37 + 11) % num_blocks."""
    return (np.arange(num_logical, dtype=np.int64) * 37 + 11) % num_blocks


def to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    _L().pkvo_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


class BlockManager:
    """model_speculative_moe_batched.mojo:789-807 (LIFO free list)."""

    def __init__(self, max_blocks: int):
        self.free_list = np.empty(max_blocks, np.int32)
        self.count = np.zeros(1, np.int32)
        _L().pkvo_bm_init(_p(self.free_list), _p(self.count), max_blocks)

    def allocate(self) -> int:
        return _L().pkvo_bm_allocate(_p(self.free_list), _p(self.count))

    def free(self, block_id: int) -> None:
        _L().pkvo_bm_free(_p(self.free_list), _p(self.count), block_id)

    @property
    def free_blocks(self) -> np.ndarray:
        return self.free_list[: int(self.count[0])].copy()


def dense_tok_off(batch: int, rows_per_seq: int) -> np.ndarray:
    """tok_off for a dense [batch][rows_per_seq] buffer where each sequence uses all rows."""
    return (np.arange(batch + 1, dtype=np.int64) * rows_per_seq).astype(np.int32)


def ragged_tok_off(n_new) -> np.ndarray:
    """tok_off for packed rows: sequence s owns n_new[s] consecutive rows."""
    n = np.maximum(np.asarray(n_new, np.int64), 0)
    return np.concatenate([[0], np.cumsum(n)]).astype(np.int32)


class CacheState:
    """CPU mirror of the device block-manager state + pools, mutated by the oracle's
    append / rollback (the engine's inline append sites and retire, see pkv_oracle.c)."""

    def __init__(self, num_layers, kv_stride, block_size, num_blocks, max_seqs, table_stride,
                 dtype=np.float32, alloc_pools=True):
        self.kv_stride = kv_stride
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.table_stride = table_stride
        self.dtype = np.dtype(dtype)
        n = num_blocks * block_size * kv_stride if alloc_pools else 0
        self.k_pools = [np.zeros(n, self.dtype) for _ in range(num_layers)]
        self.v_pools = [np.zeros(n, self.dtype) for _ in range(num_layers)]
        self.tables = np.zeros((max_seqs, table_stride), np.int32)
        self.table_lens = np.zeros(max_seqs, np.int32)
        self.bm = BlockManager(num_blocks)

    @property
    def free_list(self) -> np.ndarray:
        return self.bm.free_blocks

    def append(self, layer, pos, tok_off, k_new, v_new, max_new):
        """Ragged append: sequence s takes rows tok_off[s]..tok_off[s+1]-1 of k_new/v_new."""
        pos = np.ascontiguousarray(pos, np.int32)
        tok_off = np.ascontiguousarray(tok_off, np.int32)
        k_new = np.ascontiguousarray(k_new, self.dtype).reshape(-1, self.kv_stride)
        v_new = np.ascontiguousarray(v_new, self.dtype).reshape(-1, self.kv_stride)
        batch = pos.size
        assert tok_off.size == batch + 1
        status = np.zeros(batch, np.int32)
        _L().pkvo_append(BF16 if self.dtype == np.uint16 else F32, self.kv_stride,
                         self.block_size, _p(self.k_pools[layer]), _p(self.v_pools[layer]),
                         _p(self.tables), self.table_stride, _p(self.table_lens),
                         _p(self.bm.free_list), _p(self.bm.count), _p(pos), _p(tok_off), max_new,
                         _p(k_new), _p(v_new), k_new.shape[0], batch, _p(status))
        return status

    def rollback(self, new_len):
        """Rollback / retire of the block tables (pkvo_rollback)."""
        new_len = np.ascontiguousarray(new_len, np.int32)
        _L().pkvo_rollback(self.block_size, _p(self.tables), self.table_stride,
                           _p(self.table_lens), _p(self.bm.free_list), _p(self.bm.count),
                           _p(new_len), new_len.size)


class RingState:
    """CPU mirror of ring pools (sliding layers in the engine's default mode,
    …batched.mojo:1301-1304, :1440-1442): `num_slots` rings of `ring_size` rows per layer,
    and the kv-slot free list the scheduler pops at admission and pushes at retire
    (:2316-2318, :2487-2490, :2412-2433)."""

    def __init__(self, num_layers, kv_stride, ring_size, num_slots, dtype=np.float32):
        self.kv_stride = kv_stride
        self.ring_size = ring_size
        self.num_slots = num_slots
        self.dtype = np.dtype(dtype)
        n = num_slots * ring_size * kv_stride
        self.k_pools = [np.zeros(n, self.dtype) for _ in range(num_layers)]
        self.v_pools = [np.zeros(n, self.dtype) for _ in range(num_layers)]

    def append(self, layer, slots, pos, tok_off, k_new, v_new, max_new):
        """Ring append (pkvo_ring_append): sequence s writes rows tok_off[s]..tok_off[s+1]-1
        of k_new / v_new at ring_row(slots[s], ring_size, pos[s] + b)."""
        slots = np.ascontiguousarray(slots, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        tok_off = np.ascontiguousarray(tok_off, np.int32)
        k_new = np.ascontiguousarray(k_new, self.dtype).reshape(-1, self.kv_stride)
        v_new = np.ascontiguousarray(v_new, self.dtype).reshape(-1, self.kv_stride)
        batch = pos.size
        assert tok_off.size == batch + 1 and slots.size == batch
        status = np.zeros(batch, np.int32)
        _L().pkvo_ring_append(BF16 if self.dtype == np.uint16 else F32, self.kv_stride,
                              self.ring_size, self.num_slots, _p(self.k_pools[layer]),
                              _p(self.v_pools[layer]), _p(slots), 1, _p(pos), _p(tok_off),
                              max_new, _p(k_new), _p(v_new), k_new.shape[0], batch, _p(status))
        return status


def attend(q, k_pool, v_pool, tables, table_lens, pos, q_len, num_heads, num_kv_heads,
           head_dim, block_size, window, scale=1.0, nthreads=1, par=0, ring_size=0):
    """Batched reference attention: one paged_attention_layer call per query token
    (…batched.mojo:601-657, :3090-3123). q: [batch, q_len, Hq, D] fp32.
    ring_size > 0: ring pools, tables[s, 0] is sequence s's ring slot (:648)."""
    q = np.ascontiguousarray(q, np.float32)
    tables = np.ascontiguousarray(tables, np.int32)
    table_lens = np.ascontiguousarray(table_lens, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    batch = pos.size
    out = np.empty((batch, q_len, num_heads, head_dim), np.float32)
    rc = _L().pkvo_attend(_dtype_of(k_pool), num_heads, num_kv_heads, head_dim, block_size,
                          window, scale, _p(q), _p(k_pool), _p(v_pool), _p(tables),
                          tables.shape[1], _p(table_lens), _p(pos), q_len, batch, _p(out),
                          nthreads, par, ring_size)
    if rc != 0:
        raise RuntimeError(f"pkvo_attend rc={rc}")
    return out


def attend_f64(q, k_pool, v_pool, tables, pos, q_len, num_heads, num_kv_heads, head_dim,
               block_size, window, scale=1.0, nthreads=None, ring_size=0):
    """Exact (float64) attention for pkvo_attend's layout (test_attention.mojo:123-163)."""
    q = np.ascontiguousarray(q, np.float32)
    tables = np.ascontiguousarray(tables, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    batch = pos.size
    out = np.empty((batch, q_len, num_heads, head_dim), np.float64)
    _L().pkvo_attend_f64(_dtype_of(k_pool), num_heads, num_kv_heads, head_dim, block_size,
                         window, scale, _p(q), _p(k_pool), _p(v_pool), _p(tables),
                         tables.shape[1], _p(pos), q_len, batch, _p(out),
                         max_threads() if nthreads is None else nthreads, ring_size)
    return out


def max_rel_err(x, ref) -> float:
    """test_attention.mojo:259-266 -- max |x - ref| / (|ref| + 1e-3)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(x - ref) / (np.abs(ref) + 1e-3))) if x.size else 0.0
