"""GPU parity of ring-pool addressing (ring_size > 0): the engine's default mode for
sliding layers, where each sequence keeps its last ring_size K/V rows in a ring of its
kv slot (ring_row, attention.mojo:144-148; pools …batched.mojo:1440-1442; writes :1996,
:2625, :3111; reads :648). Ring pool bytes must match the oracle bit-exactly; attention
outputs follow tests/parity.py (1e-4 fp32 / 2e-2 bf16), and ring attention must equal
paged attention over the same keys bit-for-bit (the same kernel walks the same keys in
the same order; test_attention.mojo:500-614 asserts the same of the reference)."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, PagedKVCache, hip, lib, paged_attention_layer
from pkv.engine import make_params
from tests import parity
from tests.refcase import BLOCK_SIZE, CAPACITY, NUM_BLOCKS, Fixture

pytestmark = pytest.mark.gpu

WINDOW = 1024
RING = WINDOW + 8  # the engine's ring_size (…batched.mojo:1304)


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
def test_ring_matches_paged_single_sequence(gpu, kv_dtype):
    # test_attention.mojo:500-548 on the device, through the single-sequence drop-in.
    print(f"[ring] matches paged {kv_dtype}", flush=True)
    heads, kv_heads, head_dim = 16, 8, 256
    kv_stride = kv_heads * head_dim
    ring_size, num_slots = 1024 + 64, 3
    fx = Fixture(heads, kv_heads, head_dim, seed=77, k_scale=0.25)
    conv = O.to_bf16 if kv_dtype == BF16 else (lambda a: a)
    npdt = np.uint16 if kv_dtype == BF16 else np.float32
    k_host, v_host = conv(fx.k_pool).reshape(-1, kv_stride), conv(fx.v_pool).reshape(-1, kv_stride)
    dk, dv = hip.DeviceArray.from_numpy(k_host), hip.DeviceArray.from_numpy(v_host)
    dtab = hip.DeviceArray.from_numpy(fx.table.astype(np.int32))
    dq = hip.DeviceArray.from_numpy(fx.q)
    rk = hip.DeviceArray((num_slots * ring_size, kv_stride), npdt)
    rv = hip.DeviceArray((num_slots * ring_size, kv_stride), npdt)
    out_p = hip.DeviceArray((heads * head_dim,), np.float32)
    out_r = hip.DeviceArray((heads * head_dim,), np.float32)
    for slot in (0, 2):
        base = slot * ring_size
        for pos in (0, 1, 1023, 1024, 1087, 1088, 1089, 2000, CAPACITY - 1):
            ring_k = np.full((num_slots * ring_size, kv_stride), 9999.0, np.float32)
            ring_v = np.full((num_slots * ring_size, kv_stride), -9999.0, np.float32)
            ring_k, ring_v = conv(ring_k), conv(ring_v)
            for t in range(O.window_start(pos, WINDOW), pos + 1):
                src = fx.row_of(t) // kv_stride
                ring_k[base + t % ring_size] = k_host[src]
                ring_v[base + t % ring_size] = v_host[src]
            rk.upload(ring_k)
            rv.upload(ring_v)
            paged_attention_layer(dq, dk, dv, dtab, BLOCK_SIZE, pos, heads, kv_heads, head_dim,
                                  WINDOW, out_p, num_blocks=NUM_BLOCKS, kv_dtype=kv_dtype)
            paged_attention_layer(dq, rk, rv, None, BLOCK_SIZE, pos, heads, kv_heads, head_dim,
                                  WINDOW, out_r, ring_size, base, num_blocks=num_slots,
                                  kv_dtype=kv_dtype)
            got_r, got_p = out_r.numpy(), out_p.numpy()
            np.testing.assert_array_equal(got_r, got_p, err_msg=f"slot={slot} pos={pos}")
            ref = O.paged_attention_layer(fx.q, ring_k.reshape(-1), ring_v.reshape(-1), [],
                                          BLOCK_SIZE, pos, heads, kv_heads, head_dim, WINDOW,
                                          ring_size=ring_size, ring_base=base)
            exact = None
            if kv_dtype == F32:
                exact = O.attention_f64(fx.q, k_host.reshape(-1), v_host.reshape(-1), fx.table,
                                        BLOCK_SIZE, pos, O.window_start(pos, WINDOW), heads,
                                        kv_heads, head_dim)
            parity.check(got_r, ref, exact, bf16=kv_dtype == BF16, what=f"slot={slot} pos={pos}")


class _Mirror:
    """Oracle state beside a PagedKVCache of [ring sliding layer, paged global layer]."""

    def __init__(self, B, kv_stride, num_blocks, stride, num_slots):
        self.paged = O.CacheState(1, kv_stride, 16, num_blocks, B, stride)
        self.ring = O.RingState(1, kv_stride, RING, num_slots)


def _append_both(cache, mir, pos, n_new, rng, kv_stride, max_new):
    tok_off = O.ragged_tok_off(n_new)
    rows = max(int(tok_off[-1]), 1)
    k = rng.standard_normal((rows, kv_stride), dtype=np.float32)
    v = rng.standard_normal((rows, kv_stride), dtype=np.float32)
    dk, dv = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    st_r = cache.append(0, pos, tok_off, dk, dv, max_new, rows).numpy()
    st_p = cache.append(1, pos, tok_off, dk, dv, max_new, rows).numpy()
    want_r = mir.ring.append(0, cache.kv_slot_of, pos, tok_off, k, v, max_new)
    want_p = mir.paged.append(0, pos, tok_off, k, v, max_new)
    assert np.array_equal(st_r, want_r) and np.array_equal(st_p, want_p), (st_r, st_p)
    assert np.array_equal(cache.k_pools[0].numpy().reshape(-1), mir.ring.k_pools[0]), "ring K"
    assert np.array_equal(cache.v_pools[0].numpy().reshape(-1), mir.ring.v_pools[0]), "ring V"
    assert np.array_equal(cache.k_pools[1].numpy().reshape(-1), mir.paged.k_pools[0]), "paged K"
    snap = cache.snapshot()
    assert np.array_equal(snap["free_list"], mir.paged.free_list)
    assert np.array_equal(snap["table_lens"], mir.paged.table_lens)


def _attend_both(cache, mir, pos, q_len, rng, hq, hkv, d, what):
    B = pos.size
    q = rng.standard_normal((B, q_len, hq, d), dtype=np.float32)
    dq = hip.DeviceArray.from_numpy(q)
    out = hip.DeviceArray((B, q_len, hq, d), np.float32)
    slots = cache.kv_slot_of.reshape(-1, 1)
    zeros = np.zeros(B, np.int32)
    for layer, window in ((0, WINDOW), (1, 0)):
        cache.attend(layer, dq, pos, q_len, out)
        got = out.numpy()
        if layer == 0:
            ref = O.attend(q, mir.ring.k_pools[0], mir.ring.v_pools[0], slots, zeros, pos, q_len,
                           hq, hkv, d, 16, window, scale=cache.scale, nthreads=O.max_threads(),
                           par=1, ring_size=RING)
            exact = O.attend_f64(q, mir.ring.k_pools[0], mir.ring.v_pools[0], slots, pos, q_len,
                                 hq, hkv, d, 16, window, scale=cache.scale, ring_size=RING)
        else:
            ref = O.attend(q, mir.paged.k_pools[0], mir.paged.v_pools[0], mir.paged.tables,
                           mir.paged.table_lens, pos, q_len, hq, hkv, d, 16, window,
                           scale=cache.scale, nthreads=O.max_threads(), par=1)
            exact = O.attend_f64(q, mir.paged.k_pools[0], mir.paged.v_pools[0],
                                 mir.paged.tables, pos, q_len, hq, hkv, d, 16, window,
                                 scale=cache.scale)
        parity.check(got, ref, exact, what=f"{what} layer {layer}")


def test_ring_sliding_with_paged_global_decode_verify_retire(gpu):
    # The engine's default layout: a ring sliding layer and a paged global layer sharing
    # one scheduler. Prefill longer than the ring (only the last RING rows survive),
    # decode across ring wrap points, a 4-token verify with rejected drafts (the ring
    # keeps stale rows, the global table is rolled back), then retire / admit reusing the
    # freed kv slot. Pools, tables and free lists are compared after every append.
    rng = np.random.default_rng(21)
    hq, hkv, d = 16, 8, 256
    kv_stride = hkv * d
    B, stride, nb = 4, 260, 900
    specs = [LayerSpec(hq, hkv, d, window=WINDOW, ring_size=RING), LayerSpec(hq, hkv, d)]
    cache = PagedKVCache(specs, block_size=16, num_blocks=nb, max_seqs=B,
                         max_blocks_per_seq=stride, max_q_len=4, max_pos=stride * 16 - 1,
                         scale=0.0625, num_kv_slots=B + 1)
    mir = _Mirror(B, kv_stride, nb, stride, B + 1)
    cache.admit(range(B))
    assert list(cache.kv_slot_of) == [0, 1, 2, 3]  # LIFO list [4, 3, 2, 1, 0]
    ctx = np.array([1028, 2060, 3095, 500], np.int32)
    print("[ring] prefill", flush=True)
    _append_both(cache, mir, np.zeros(B, np.int32), ctx, rng, kv_stride, int(ctx.max()))
    pos = ctx.copy()
    for step in range(6):  # seq 2 wraps at step 1, seqs 0 and 1 at step 4
        print(f"[ring] decode step {step}", flush=True)
        _append_both(cache, mir, pos, np.ones(B, np.int32), rng, kv_stride, 1)
        _attend_both(cache, mir, pos, 1, rng, hq, hkv, d, f"decode {step}")
        pos += 1
    print("[ring] verify", flush=True)
    _append_both(cache, mir, pos, np.full(B, 4, np.int32), rng, kv_stride, 4)
    _attend_both(cache, mir, pos, 4, rng, hq, hkv, d, "verify")
    acc = np.array([0, 3, 1, 2], np.int32)
    pos += acc + 1
    cache.rollback(pos)
    mir.paged.rollback(pos)
    snap = cache.snapshot()
    assert np.array_equal(snap["free_list"], mir.paged.free_list)
    print("[ring] decode after verify", flush=True)
    _append_both(cache, mir, pos, np.ones(B, np.int32), rng, kv_stride, 1)
    _attend_both(cache, mir, pos, 1, rng, hq, hkv, d, "after verify")
    pos += 1
    print("[ring] retire / admit", flush=True)
    cache.retire([1])
    mir.paged.rollback(np.array([-1, 0, -1, -1], np.int32))
    assert cache.free_kv_slots[-1] == 1
    cache.admit([1])
    assert cache.kv_slot_of[1] == 1  # the freed kv slot is reused
    pos[1] = 0
    n_new = np.array([0, 300, 0, 0], np.int32)
    _append_both(cache, mir, pos, n_new, rng, kv_stride, 300)
    pos[1] = 300
    _append_both(cache, mir, pos, np.ones(B, np.int32), rng, kv_stride, 1)
    _attend_both(cache, mir, pos, 1, rng, hq, hkv, d, "after admit")
    cache.free()


def _ring_case(rng, B, q_len, pos, hq, hkv, d, window, ring_size, kv_dtype, slots, num_slots):
    kvs = hkv * d
    k = rng.standard_normal(num_slots * ring_size * kvs, dtype=np.float32)
    v = rng.standard_normal(num_slots * ring_size * kvs, dtype=np.float32)
    if kv_dtype == BF16:
        k, v = O.to_bf16(k), O.to_bf16(v)
    q = rng.standard_normal((B, q_len, hq, d), dtype=np.float32)
    p = make_params(LayerSpec(hq, hkv, d, window, kv_dtype, ring_size), 16, num_slots, 0.0625)
    max_pos = int(pos.max()) + q_len - 1
    ws_bytes = lib.load().pkv_workspace_size(ctypes.byref(p), B, q_len, max_pos)
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    dk, dv = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    dslots = hip.DeviceArray.from_numpy(np.asarray(slots, np.int32))
    dq, dpos = hip.DeviceArray.from_numpy(q), hip.DeviceArray.from_numpy(pos)
    out = hip.DeviceArray((B, q_len, hq, d), np.float32)
    lib.call("pkv_attend", None, ctypes.byref(p), dq.ptr, dk.ptr, dv.ptr, dslots.ptr, 1,
             dpos.ptr, q_len, B, max_pos, out.ptr, ws.ptr, ws.nbytes)
    return out.numpy(), (q, k, v)


@pytest.mark.parametrize("geom,q_len,window,ring_size,kv_dtype", [
    ((16, 2, 512), 1, 600, 640, F32),   # head_dim 512: the chunk kernel
    ((16, 8, 256), 8, WINDOW, RING, F32),  # 16 rows per kv head: the chunk kernel
    ((16, 8, 256), 4, WINDOW, RING, BF16),  # stream kernel, bf16 ring
    ((16, 8, 256), 2, 0, 700, F32),      # full causal over a ring that holds everything
], ids=["d512", "rows16", "bf16-verify", "causal"])
def test_ring_attend_kernels(gpu, geom, q_len, window, ring_size, kv_dtype):
    print(f"[ring] attend {geom} q_len={q_len} window={window} ring={ring_size}", flush=True)
    rng = np.random.default_rng(q_len * 7 + geom[2])
    hq, hkv, d = geom
    B, num_slots = 5, 6
    slots = np.array([4, 0, 5, 2, 1], np.int32)
    if window > 0:
        pos = np.array([0, 30, window - 5, window + 400, 3 * ring_size + 17], np.int32)
    else:
        pos = np.array([0, 30, 300, ring_size - q_len - 3, ring_size - q_len], np.int32)
    got, (q, k, v) = _ring_case(rng, B, q_len, pos, hq, hkv, d, window, ring_size, kv_dtype,
                                slots, num_slots)
    tab = slots.reshape(-1, 1)
    zeros = np.zeros(B, np.int32)
    ref = O.attend(q, k, v, tab, zeros, pos, q_len, hq, hkv, d, 16, window, scale=0.0625,
                   nthreads=O.max_threads(), par=1, ring_size=ring_size)
    exact = None
    if kv_dtype == F32:
        exact = O.attend_f64(q, k, v, tab, pos, q_len, hq, hkv, d, 16, window, scale=0.0625,
                             ring_size=ring_size)
    parity.check(got, ref, exact, bf16=kv_dtype == BF16, what="ring attend")


def test_ring_bad_slot_and_overlong_span(gpu):
    # A kv slot outside the pool, or a call whose keys would not all be in the ring (the
    # reference aborts, attention.mojo:265-266), gives NaN outputs and reads nothing;
    # a ring append to a bad slot writes nothing and reports PKV_SEQ_BAD_BLOCK.
    print("[ring] bad slot / overlong span", flush=True)
    rng = np.random.default_rng(5)
    hq, hkv, d, ring_size, num_slots = 16, 8, 256, 1026, 3
    q_len = 4
    slots = np.array([0, 7, 2], np.int32)
    pos = np.array([100, 100, 2000], np.int32)  # seq 2: 1027 keys > ring 1026
    got, _ = _ring_case(rng, 3, q_len, pos, hq, hkv, d, WINDOW, ring_size, F32, slots,
                        num_slots)
    assert np.all(np.isfinite(got[0]))
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))
    p = make_params(LayerSpec(hq, hkv, d, WINDOW, F32, ring_size), 16, num_slots, 1.0)
    kvs = hkv * d
    pool = hip.DeviceArray((num_slots * ring_size * kvs,), np.float32, zero=True)
    k_new = hip.DeviceArray.from_numpy(np.ones((3, kvs), np.float32))
    dslots = hip.DeviceArray.from_numpy(slots)
    dpos = hip.DeviceArray.from_numpy(np.array([5, 5, 5], np.int32))
    doff = hip.DeviceArray.from_numpy(O.dense_tok_off(3, 1))
    status = hip.DeviceArray((3,), np.int32, zero=True)
    lib.call("pkv_append", None, ctypes.byref(p), pool.ptr, pool.ptr, dslots.ptr, 1, None, None,
             None, dpos.ptr, doff.ptr, 1, k_new.ptr, k_new.ptr, 3, 3, status.ptr)
    assert list(status.numpy()) == [lib.PKV_SEQ_OK, lib.PKV_SEQ_BAD_BLOCK, lib.PKV_SEQ_OK]
    host = pool.numpy().reshape(num_slots * ring_size, kvs)
    written = np.flatnonzero(host.any(axis=1))
    assert list(written) == [5, 2 * ring_size + 5]
