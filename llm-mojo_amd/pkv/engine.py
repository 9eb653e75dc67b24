"""Host-side mirror of the reference engine's paged-KV operator surface over libpkv.

Reference host code (phildrip/llm-mojo, Mojo):
  - attention_window_start / ring_row      attention.mojo:135-148
  - paged_attention_layer                  attention.mojo:240-294
  - BlockManager / Sequence state          model_speculative_moe_batched.mojo:789-845
  - pools, one table per sequence shared by all layers   :1427-1451, :1995-1998
  - inline KV append                       :1984-2001 (and the prefill/verify sites)
  - retire (free table ascending)          :3626-3628
  - ring pools for sliding layers, kv slots :1301-1304, :1440-1442, :2316-2318, :2487-2490

Here the block-manager state (tables, lengths, LIFO free list) lives in device memory
and every mutation is a libpkv kernel, so a batched decode step never round-trips
through the host. Numbers on the host side are only what the caller feeds in
(positions, token counts, new lengths).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import hip, lib

F32 = "f32"
BF16 = "bf16"
_DTYPES = {F32: lib.PKV_DTYPE_F32, BF16: lib.PKV_DTYPE_BF16}
_NP_KV = {F32: np.float32, BF16: np.uint16}  # bf16 is carried as its 16-bit pattern


def attention_window_start(pos: int, window: int) -> int:
    """First key position attended by the query at `pos` (attention.mojo:135-141)."""
    if window <= 0:
        return 0
    start = pos - window + 1
    return start if start > 0 else 0


def ring_row(slot: int, ring_size: int, t: int) -> int:
    """Physical row of token t in ring slot `slot` (attention.mojo:144-148)."""
    return slot * ring_size + t % ring_size


@dataclass(frozen=True)
class LayerSpec:
    """Geometry of one attention layer's pools (Gemma-4: sliding 16/8/256 window 1024,
    global 16/2/512 full causal; the benchmark configs use 16/8/256 for both).

    ring_size > 0 keeps the layer's K/V in one ring of ring_size rows per kv slot instead
    of pages -- the engine's default for sliding layers, ring_size = window + 8
    (…batched.mojo:1304)."""

    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 256
    window: int = 0
    kv_dtype: str = F32
    ring_size: int = 0

    @property
    def kv_stride(self) -> int:
        return self.num_kv_heads * self.head_dim


def make_params(spec: LayerSpec, block_size: int, num_blocks: int,
                scale: float = 1.0) -> lib.PkvParams:
    """pkv_params for one layer; for a ring layer num_blocks is the number of kv slots."""
    p = lib.PkvParams()
    p.num_heads = spec.num_heads
    p.num_kv_heads = spec.num_kv_heads
    p.head_dim = spec.head_dim
    p.block_size = block_size
    p.num_blocks = num_blocks
    p.window = spec.window
    p.scale = scale
    p.kv_dtype = _DTYPES[spec.kv_dtype]
    p.ring_size = spec.ring_size
    p.reserved = 0
    return p


def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, hip.DeviceArray):
        return x.ptr
    return int(x)


class PagedKVCache:
    """Device-resident paged KV cache: per-layer K/V pools of `num_blocks` blocks of
    `block_size` tokens, one block table per sequence slot shared by every layer, and
    the BlockManager's LIFO free list.

    Pools are zero-filled at creation like the reference's (…batched.mojo:1444-1447);
    the free list starts as [0 .. num_blocks-1] with every block free (:795-799).

    Ring layers (LayerSpec.ring_size > 0) hold `num_kv_slots` rings of ring_size rows
    instead (:1440-1442). A sequence slot takes a kv slot at admission from a LIFO list
    initialised to [num_kv_slots-1 .. 0] (:2316-2318, :2487-2490) and returns it at
    retire (:2412-2433); `kv_slots` (device int32 [max_seqs]) holds the assignment and
    is what ring-layer calls pass as their one-entry "table" per sequence."""

    def __init__(self, layers: list[LayerSpec], *, block_size: int, num_blocks: int,
                 max_seqs: int, max_blocks_per_seq: int, max_q_len: int = 1,
                 max_pos: int | None = None, scale: float = 1.0, stream: hip.Stream | None = None,
                 num_kv_slots: int | None = None):
        lib.load()
        self.layers = list(layers)
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.max_seqs = max_seqs
        self.table_stride = max_blocks_per_seq
        self.max_q_len = max_q_len
        self.max_pos = max_pos if max_pos is not None else max_blocks_per_seq * block_size - 1
        self.scale = scale
        self.stream = stream
        self.num_kv_slots = max_seqs if num_kv_slots is None else num_kv_slots
        self.params = [make_params(s, block_size,
                                   self.num_kv_slots if s.ring_size > 0 else num_blocks, scale)
                       for s in self.layers]
        self.k_pools, self.v_pools = [], []
        for s in self.layers:
            if s.ring_size > 0:
                shape = (self.num_kv_slots, s.ring_size, s.num_kv_heads, s.head_dim)
            else:
                shape = (num_blocks, block_size, s.num_kv_heads, s.head_dim)
            self.k_pools.append(hip.DeviceArray(shape, _NP_KV[s.kv_dtype], zero=True))
            self.v_pools.append(hip.DeviceArray(shape, _NP_KV[s.kv_dtype], zero=True))
        self.free_kv_slots = list(range(self.num_kv_slots - 1, -1, -1))
        self.kv_slot_of = np.full(max_seqs, -1, np.int32)
        self.kv_slots = hip.DeviceArray.from_numpy(self.kv_slot_of)
        self.tables = hip.DeviceArray((max_seqs, max_blocks_per_seq), np.int32, zero=True)
        self.table_lens = hip.DeviceArray((max_seqs,), np.int32, zero=True)
        self.free_list = hip.DeviceArray.from_numpy(np.arange(num_blocks, dtype=np.int32))
        self.free_count = hip.DeviceArray.from_numpy(np.array([num_blocks], dtype=np.int32))
        self.status = hip.DeviceArray((max_seqs,), np.int32, zero=True)
        ws = 0
        for p in self.params:
            need = lib.load().pkv_workspace_size(ctypes.byref(p), max_seqs, max_q_len,
                                                 self.max_pos)
            if need == 0:
                raise lib.PkvError(-1, "pkv_workspace_size", lib.load().pkv_last_error().decode())
            ws = max(ws, need)
        self.workspace = hip.DeviceArray((ws,), np.uint8, zero=True)
        # Small host->device staging buffers for per-call integer arguments.
        self._i32_a = hip.DeviceArray((max_seqs,), np.int32, zero=True)
        self._i32_b = hip.DeviceArray((max_seqs + 1,), np.int32, zero=True)

    # -------------------------------------------------------------- helpers
    def _stream(self):
        return self.stream.handle if self.stream else None

    def _ints(self, x, staging: hip.DeviceArray, n: int):
        """Device pointer for an int32[n] argument given as numpy/list or device array."""
        if isinstance(x, (np.ndarray, list, tuple)):
            arr = np.ascontiguousarray(np.asarray(x, dtype=np.int32).reshape(-1))
            if arr.size != n:
                raise ValueError(f"expected {n} ints, got {arr.size}")
            staging.upload_at(0, arr)
            return staging.ptr
        return _ptr(x)

    def _tables_of(self, layer: int):
        """(tables, stride) a layer's calls pass: block tables, or the kv-slot array."""
        if self.layers[layer].ring_size > 0:
            return self.kv_slots.ptr, 1
        return self.tables.ptr, self.table_stride

    # ------------------------------------------------------------- kv slots
    def admit(self, slots) -> None:
        """Gives each sequence slot a kv slot (ring layers) from the LIFO list
        (…batched.mojo:2487-2490). No-op for slots that already hold one."""
        for s in slots:
            if self.kv_slot_of[s] < 0:
                if not self.free_kv_slots:
                    raise RuntimeError("no free kv slot (num_kv_slots < active sequences)")
                self.kv_slot_of[s] = self.free_kv_slots.pop()
        self.kv_slots.upload_at(0, self.kv_slot_of)

    def _release(self, slots) -> None:
        """Returns the kv slots of retired sequences (…batched.mojo:2412-2433)."""
        for s in slots:
            if self.kv_slot_of[s] >= 0:
                self.free_kv_slots.append(int(self.kv_slot_of[s]))
                self.kv_slot_of[s] = -1
        self.kv_slots.upload_at(0, self.kv_slot_of)

    # ------------------------------------------------------------ operators
    def append(self, layer: int, pos, tok_off, k_new, v_new, max_new: int, total_rows: int,
               batch: int | None = None):
        """KV append for `batch` sequence slots (K1). pos: int32[batch]; tok_off:
        int32[batch + 1] (numpy or device) -- slot s appends rows tok_off[s] ..
        tok_off[s+1]-1 of k_new / v_new (device [total_rows][kv_stride], pool dtype) at
        positions pos[s], pos[s] + 1, ... Returns the device status array (PKV_SEQ_*).
        A ring layer writes into each sequence's ring and allocates no block."""
        b = batch or self.max_seqs
        p = self.params[layer]
        tables, stride = self._tables_of(layer)
        lib.call("pkv_append", self._stream(), ctypes.byref(p), self.k_pools[layer].ptr,
                 self.v_pools[layer].ptr, tables, stride,
                 self.table_lens.ptr, self.free_list.ptr, self.free_count.ptr,
                 self._ints(pos, self._i32_a, b), self._ints(tok_off, self._i32_b, b + 1),
                 max_new, _ptr(k_new), _ptr(v_new), total_rows, b, self.status.ptr)
        return self.status

    def append_qkv(self, layer: int, pos, tok_off, q, k, v, q_norm_w, k_norm_w, q_out,
                   max_new: int, total_rows: int, is_global: bool, q_out_dtype: str = F32,
                   batch: int | None = None):
        """Producer step + append (K1'): per-head rms_norm of Q / K (weights q_norm_w,
        k_norm_w), rms_norm_noscale of V (v=None: V := K as read), RoPE of Q and K at each
        token's position, then the K / V rows are appended as in append(). q, k, v, the
        weights and q_out are device arrays (q_out in q_out_dtype). Returns the status."""
        b = batch or self.max_seqs
        p = self.params[layer]
        tables, stride = self._tables_of(layer)
        lib.call("pkv_append_qkv", self._stream(), ctypes.byref(p), int(bool(is_global)),
                 self.k_pools[layer].ptr, self.v_pools[layer].ptr, tables, stride,
                 self.table_lens.ptr, self.free_list.ptr, self.free_count.ptr,
                 self._ints(pos, self._i32_a, b), self._ints(tok_off, self._i32_b, b + 1),
                 max_new, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_w), _ptr(k_norm_w),
                 _ptr(q_out), _DTYPES[q_out_dtype], total_rows, b, self.status.ptr)
        return self.status

    def attend(self, layer: int, q, pos, q_len: int, out, batch: int | None = None,
               max_pos: int | None = None):
        """Paged attention (K2): q/out device fp32 [batch][q_len][Hq][D]; query j of
        sequence s at position pos[s] + j."""
        b = batch or self.max_seqs
        p = self.params[layer]
        tables, stride = self._tables_of(layer)
        lib.call("pkv_attend", self._stream(), ctypes.byref(p), _ptr(q),
                 self.k_pools[layer].ptr, self.v_pools[layer].ptr, tables,
                 stride, self._ints(pos, self._i32_a, b), q_len, b,
                 self.max_pos if max_pos is None else max_pos, _ptr(out), self.workspace.ptr,
                 self.workspace.nbytes)

    def append_attend(self, layer: int, pos, tok_off, k_new, v_new, max_new: int,
                      total_rows: int, q, q_len: int, out, batch: int | None = None,
                      max_pos: int | None = None):
        """append() then attend() over the same pos in one call (pkv_append_attend): where
        the stream kernel's vector path covers the call, its launch also writes the new
        rows into the pool, saving the scatter launch. Same results as the two calls.
        Returns the device status array."""
        b = batch or self.max_seqs
        p = self.params[layer]
        tables, stride = self._tables_of(layer)
        lib.call("pkv_append_attend", self._stream(), ctypes.byref(p), self.k_pools[layer].ptr,
                 self.v_pools[layer].ptr, tables, stride, self.table_lens.ptr,
                 self.free_list.ptr, self.free_count.ptr, self._ints(pos, self._i32_a, b),
                 self._ints(tok_off, self._i32_b, b + 1), max_new, _ptr(k_new), _ptr(v_new),
                 total_rows, self.status.ptr, _ptr(q), q_len, b,
                 self.max_pos if max_pos is None else max_pos, _ptr(out), self.workspace.ptr,
                 self.workspace.nbytes)
        return self.status

    def verify(self, layer: int, q, pos, q_lens, max_q_len: int, out, batch: int | None = None,
               max_pos: int | None = None):
        """Verify attention with a query count per sequence (pkv_verify): q / out device
        fp32 [batch][max_q_len][Hq][D]; sequence s has q_lens[s] queries at positions
        pos[s] + j, and its rows past q_lens[s] are not written."""
        b = batch or self.max_seqs
        p = self.params[layer]
        tables, stride = self._tables_of(layer)
        lib.call("pkv_verify", self._stream(), ctypes.byref(p), _ptr(q),
                 self.k_pools[layer].ptr, self.v_pools[layer].ptr, tables, stride,
                 self._ints(pos, self._i32_a, b), self._ints(q_lens, self._i32_b, b), max_q_len,
                 b, self.max_pos if max_pos is None else max_pos, _ptr(out), self.workspace.ptr,
                 self.workspace.nbytes)

    def attend_sparse(self, layer: int, q, keys, key_off, max_keys: int, out,
                      batch: int | None = None):
        """Sparse paged attention over explicit key lists (K2', LSA): q / out device fp32
        [batch][Hq][D]; sequence s attends key positions keys[key_off[s] .. key_off[s+1])
        (device int32 arrays, e.g. from lsa_expand_buckets) of its table."""
        b = batch or self.max_seqs
        p = self.params[layer]
        need = lib.load().pkv_sparse_workspace_size(ctypes.byref(p), b, max_keys)
        if need == 0:
            raise lib.PkvError(-1, "pkv_sparse_workspace_size", lib.load().pkv_last_error().decode())
        if need > self.workspace.nbytes:
            self.workspace.free()
            self.workspace = hip.DeviceArray((need,), np.uint8, zero=True)
        lib.call("pkv_attend_sparse", self._stream(), ctypes.byref(p), _ptr(q),
                 self.k_pools[layer].ptr, self.v_pools[layer].ptr, self.tables.ptr,
                 self.table_stride, _ptr(keys), self._ints(key_off, self._i32_b, b + 1),
                 max_keys, b, _ptr(out), self.workspace.ptr, self.workspace.nbytes)

    def prefill(self, layer: int, q, pos, q_off, max_q: int, out, batch: int | None = None,
                max_pos: int | None = None):
        """Chunked-prefill attention (K3, bf16 pools): q bf16 [rows][Hq][D] (device),
        out fp32 [rows][Hq][D]; sequence s owns rows q_off[s] .. q_off[s+1]-1 at positions
        pos[s], pos[s] + 1, ... and attends causally over its prefix and the chunk."""
        b = batch or self.max_seqs
        p = self.params[layer]
        lib.call("pkv_prefill", self._stream(), ctypes.byref(p), _ptr(q),
                 self.k_pools[layer].ptr, self.v_pools[layer].ptr, self.tables.ptr,
                 self.table_stride, self._ints(pos, self._i32_a, b),
                 self._ints(q_off, self._i32_b, b + 1), max_q, b,
                 self.max_pos if max_pos is None else max_pos, _ptr(out))

    def rollback(self, new_len, batch: int | None = None, status=None):
        """Truncate tables to ceil(new_len / block_size) blocks, freeing the tail in
        ascending logical order (K5). new_len[s] < 0 leaves slot s alone; 0 retires it."""
        b = batch or self.max_seqs
        p = next((q for q, s in zip(self.params, self.layers) if s.ring_size == 0), None)
        if p is None:
            return self.status  # ring layers only: no block tables to truncate
        lib.call("pkv_rollback", self._stream(), ctypes.byref(p), self.tables.ptr,
                 self.table_stride, self.table_lens.ptr, self.free_list.ptr,
                 self.free_count.ptr, self._ints(new_len, self._i32_a, b), b,
                 _ptr(status) if status is not None else self.status.ptr)
        return self.status

    def retire(self, slots, batch: int | None = None):
        """Free every block of the given slots (…batched.mojo:3626-3628) and return
        their kv slots."""
        b = batch or self.max_seqs
        nl = np.full(b, -1, dtype=np.int32)
        nl[list(slots)] = 0
        self._release(slots)
        return self.rollback(nl, b)

    # ---------------------------------------------------------------- state
    def snapshot(self) -> dict:
        hip.synchronize()
        fc = int(self.free_count.numpy()[0])
        return {
            "tables": self.tables.numpy(),
            "table_lens": self.table_lens.numpy(),
            "free_list": self.free_list.numpy()[:fc].copy(),
            "free_count": fc,
        }

    def free(self):
        for a in self.k_pools + self.v_pools:
            a.free()
        for a in (self.tables, self.table_lens, self.free_list, self.free_count, self.status,
                  self.workspace, self._i32_a, self._i32_b, self.kv_slots):
            a.free()


def q4_matmul(w_packed, scales, x, out, c_in: int, c_out: int, batch: int, workspace=None,
              stream: hip.Stream | None = None):
    """Wo projection (q4_matmul_vec, moe_kernels.mojo:59-163) for `batch` vectors: out
    [batch][c_out] = x [batch][c_in] times the Q4_0 matrix (w_packed [c_out][c_in/2] uint8,
    scales [c_out][c_in/32] fp32); all device arrays, w_packed and x 16-byte aligned (device
    allocations are). A workspace passed in must have been zero-filled before its first use
    (each call leaves it so). Returns the workspace used."""
    L = lib.load()
    need = L.pkv_q4_matmul_workspace_size(c_in, c_out, batch)
    if need == 0:
        raise lib.PkvError(lib.PKV_ERR_INVALID, "pkv_q4_matmul_workspace_size", "invalid sizes")
    ws = workspace
    if ws is None or ws.nbytes < need:
        ws = hip.DeviceArray((need,), np.uint8, zero=True)  # zero-filled before first use
    lib.call("pkv_q4_matmul", stream.handle if stream else None, _ptr(w_packed), _ptr(scales),
             _ptr(x), c_in, c_out, batch, _ptr(out), ws.ptr, ws.nbytes)
    return ws


def lsa_expand_buckets(picked, sizes, members, pos: int, top_k: int, sink_size: int,
                       window_size: int) -> np.ndarray:
    """Key list of one LSA query (LSALayerIndex.expand_buckets, lsa_core.mojo:573-604):
    members of the picked buckets, in order, that lie in [sink_size, window_start), at most
    top_k of them; then the window [window_start, pos], window_start = max(0, pos + 1 -
    window_size); then the sinks [0, min(sink_size, window_start, pos + 1)).
    members: [buckets][bucket_cap] positions, sizes: [buckets]."""
    window_start = max(0, pos + 1 - window_size)
    sel: list[int] = []
    for b in picked:
        for tok in members[b][: int(sizes[b])]:
            if sink_size <= tok < window_start:
                sel.append(int(tok))
                if len(sel) >= top_k:
                    break
        if len(sel) >= top_k:
            break
    sel.extend(range(window_start, pos + 1))
    sel.extend(range(min(sink_size, window_start, pos + 1)))
    return np.asarray(sel, np.int32)


class LSABucketCache:
    """The bucket caches of the engine's LSA indices (one LSALayerIndex per kv slot and
    global-layer group, model_speculative_moe_batched.mojo:1885-1888, :632) held in device
    memory: per instance the member counts and member positions of its buckets
    (lsa_core.mojo:222-233), its closed cluster blocks and tokens appended. expand() is
    expand_buckets for a batch of queries, writing pkv_attend_sparse's key lists on the
    device; rollback_to() is rollback_to / reset for a batch of instances. Filling a block's
    buckets (Ward clustering on block close) and picking buckets stay with the index on the
    host, which copies a closed block in with load_block()."""

    BUCKET_CAP = 32
    BLOCK_BUCKETS = 32

    def __init__(self, num_indices: int, max_capacity: int = 131072):
        self.num_indices = num_indices
        self.max_capacity = max_capacity
        self.max_buckets = (max_capacity + 511) // 512 * self.BLOCK_BUCKETS
        self.sizes = hip.DeviceArray((num_indices, self.max_buckets), np.int32, zero=True)
        self.members = hip.DeviceArray((num_indices, self.max_buckets, self.BUCKET_CAP),
                                       np.int32, zero=True)
        self.closed_blocks = hip.DeviceArray((num_indices,), np.int32, zero=True)
        self.total_tokens = hip.DeviceArray((num_indices,), np.int32, zero=True)
        self.workspace = None

    def load_block(self, index: int, block: int, sizes, members) -> None:
        """Copy one closed cluster block's 32 bucket sizes and [32][32] member rows in."""
        sizes = np.ascontiguousarray(sizes, np.int32).reshape(self.BLOCK_BUCKETS)
        members = np.ascontiguousarray(members, np.int32).reshape(self.BLOCK_BUCKETS,
                                                                   self.BUCKET_CAP)
        b0 = (index * self.max_buckets + block * self.BLOCK_BUCKETS)
        self.sizes.upload_at(b0 * 4, sizes)
        self.members.upload_at(b0 * self.BUCKET_CAP * 4, members)

    @staticmethod
    def max_keys(top_k: int, sink_size: int, window_size: int) -> int:
        """Longest list expand() builds (pkv_lsa_max_keys)."""
        return lib.load().pkv_lsa_max_keys(top_k, sink_size, window_size)

    def expand(self, index_ids, picked, n_picked, pos, top_k: int, sink_size: int,
               window_size: int, keys=None, key_off=None, status=None,
               stream: hip.Stream | None = None):
        """expand_buckets (lsa_core.mojo:568-604) for sequence s = 0..batch-1 on instance
        index_ids[s], buckets picked[s][:n_picked[s]]; device int32 arrays. Returns the
        device arrays (keys, key_off, status) for pkv_attend_sparse."""
        batch = index_ids.shape[0]
        per = self.max_keys(top_k, sink_size, window_size)
        if per < 0:
            raise lib.PkvError(lib.PKV_ERR_INVALID, "pkv_lsa_max_keys", "overflow")
        if keys is None:
            keys = hip.DeviceArray((batch * per,), np.int32)
        if key_off is None:
            key_off = hip.DeviceArray((batch + 1,), np.int32)
        if status is None:
            status = hip.DeviceArray((batch,), np.int32)
        stride = picked.shape[1] if len(picked.shape) > 1 else 0
        need = lib.load().pkv_lsa_expand_workspace_size(batch, top_k, sink_size, window_size)
        if self.workspace is None or self.workspace.nbytes < need:
            self.workspace = hip.DeviceArray((need,), np.uint8)
        lib.call("pkv_lsa_expand", stream.handle if stream else None, _ptr(index_ids),
                 _ptr(picked), stride, _ptr(n_picked), _ptr(pos), top_k, sink_size,
                 window_size, batch, self.sizes.ptr, self.members.ptr, self.num_indices,
                 self.max_buckets, _ptr(keys), _ptr(key_off), keys.nbytes // 4, _ptr(status),
                 self.workspace.ptr, self.workspace.nbytes)
        return keys, key_off, status

    def rollback_to(self, index_ids, target_tokens, stream: hip.Stream | None = None) -> None:
        """rollback_to (lsa_core.mojo:287-303; reset for targets <= 0) of instance
        index_ids[k] to target_tokens[k], entries in order (device int32 arrays)."""
        lib.call("pkv_lsa_rollback", stream.handle if stream else None, _ptr(index_ids),
                 _ptr(target_tokens), index_ids.shape[0], self.num_indices, self.max_capacity,
                 self.max_buckets, self.closed_blocks.ptr, self.total_tokens.ptr,
                 self.sizes.ptr)


def paged_attention_layer(q, k_pool, v_pool, block_table, block_size: int, pos: int,
                          num_heads: int, num_kv_heads: int, head_dim: int, window: int,
                          attn_out, ring_size: int = 0, ring_base: int = 0, *,
                          num_blocks: int, kv_dtype: str = F32, workspace=None,
                          stream: hip.Stream | None = None) -> None:
    """Single-sequence drop-in with the reference's argument list (attention.mojo:240-256).

    All buffers are device memory. The reference's `scores` / `rows` scratch becomes
    `workspace` (allocated here when not given); num_blocks / kv_dtype bound the pool."""
    L = lib.load()
    ws = workspace
    if ws is None:
        p = make_params(LayerSpec(num_heads, num_kv_heads, head_dim, window, kv_dtype),
                        block_size, num_blocks)
        need = L.pkv_workspace_size(ctypes.byref(p), 1, 1, max(pos, 0))
        ws = hip.DeviceArray((max(need, 256),), np.uint8, zero=True)
    lib.call("pkv_paged_attention_layer", stream.handle if stream else None, _ptr(q),
             _ptr(k_pool), _ptr(v_pool), _ptr(block_table), block_size, pos, num_heads,
             num_kv_heads, head_dim, window, _ptr(attn_out), ring_size, ring_base, num_blocks,
             _DTYPES[kv_dtype], ws.ptr, ws.nbytes)
