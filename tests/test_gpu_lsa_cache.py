"""GPU parity of the device LSA bucket cache: pkv_lsa_expand against the oracle's
expand_buckets restatement (lsa_core.mojo:568-604), sequence by sequence and bit-exact;
pkv_lsa_expand feeding pkv_attend_sparse against the oracle's sparse attention; and
pkv_lsa_rollback against the oracle's rollback_to / reset (lsa_core.mojo:281-303) applied
entry by entry. Integer work: every comparison is exact (the attention by tests/parity.py)."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from pkv import F32, LayerSpec, LSABucketCache, hip, lib
from pkv.engine import make_params
from tests import parity

pytestmark = pytest.mark.gpu

CAP = 32


def _fill(rng, num_indices, max_capacity, max_pos):
    """Random bucket caches: every closed block's 32 buckets get 0..32 member positions."""
    max_buckets = (max_capacity + 511) // 512 * 32
    sizes = rng.integers(0, CAP + 1, (num_indices, max_buckets)).astype(np.int32)
    members = rng.integers(0, max_pos, (num_indices, max_buckets, CAP)).astype(np.int32)
    return sizes, members


def _upload(cache, sizes, members):
    cache.sizes.upload_at(0, sizes)
    cache.members.upload_at(0, members)


def _expected(sizes, members, ids, picked, n_picked, pos, top_k, sink, window, nidx, maxb):
    keys, off, status = [], [0], []
    for s in range(len(ids)):
        bad = not (0 <= ids[s] < nidx)
        n = int(n_picked[s])
        if n < 0 or n > picked.shape[1]:
            bad, n = True, max(0, min(n, picked.shape[1]))
        if bad and not (0 <= ids[s] < nidx):
            sel = O.lsa_expand_buckets([], np.zeros(1), np.zeros((1, CAP)), int(pos[s]), top_k,
                                       sink, window)
        else:
            pk = [int(b) for b in picked[s, :n]]
            # an out-of-range bucket counts as empty; give it one empty slot past the cache
            ext_sizes = np.concatenate([sizes[ids[s]], [0]])
            ext_members = np.concatenate([members[ids[s]], np.zeros((1, CAP), np.int32)])
            pk = [b if 0 <= b < maxb else maxb for b in pk]
            sel = O.lsa_expand_buckets(pk, ext_sizes, ext_members, int(pos[s]), top_k, sink, window)
            # the flag covers the buckets the reference loop visits before its list is full
            ws = max(0, int(pos[s]) + 1 - window)
            got = 0
            for j, b in enumerate(pk):
                if j > 0 and got >= top_k:
                    break
                if b == maxb:
                    bad = True
                    continue
                kept = [t for t in ext_members[b][:ext_sizes[b]] if sink <= t < ws]
                got += min(len(kept), max(top_k - got, 1))
        keys.append(sel.astype(np.int32))
        off.append(off[-1] + sel.size)
        status.append(lib.PKV_SEQ_BAD_INDEX if bad else lib.PKV_SEQ_OK)
    return np.concatenate(keys), np.asarray(off, np.int32), np.asarray(status, np.int32)


def _expand(cache, ids, picked, n_picked, pos, top_k, sink, window):
    dev = [hip.DeviceArray.from_numpy(np.ascontiguousarray(a, np.int32))
           for a in (ids, picked, n_picked, pos)]
    keys, off, status = cache.expand(*dev, top_k, sink, window)
    n = off.numpy()
    return keys.numpy()[:n[-1]], n, status.numpy()


@pytest.mark.parametrize("top_k,sink,window", [(64, 4, 16), (128, 4, 256), (0, 4, 16),
                                               (-1, 0, 0), (5, 600, 16)],
                         ids=["k64-w16", "k128-w256", "k0", "k-1-nowindow", "sinks-past-window"])
def test_expand_matches_oracle(gpu, top_k, sink, window):
    print(f"[lsa-cache] expand top_k={top_k} sink={sink} window={window}", flush=True)
    rng = np.random.default_rng(abs(top_k) * 7 + sink + window)
    nidx, max_capacity = 10, 4096
    cache = LSABucketCache(nidx, max_capacity)
    sizes, members = _fill(rng, nidx, max_capacity, 3000)
    _upload(cache, sizes, members)
    B, stride = 70, 8  # more sequences than the kernel's 16 waves
    ids = rng.integers(0, nidx, B)
    n_picked = rng.integers(0, stride + 1, B)
    picked = rng.integers(0, cache.max_buckets, (B, stride))
    pos = rng.integers(0, 3000, B)
    pos[:3] = [0, 1, 2999]
    got_keys, got_off, got_status = _expand(cache, ids, picked, n_picked, pos, top_k, sink, window)
    want_keys, want_off, want_status = _expected(sizes, members, ids, picked, n_picked, pos, top_k,
                                                 sink, window, nidx, cache.max_buckets)
    np.testing.assert_array_equal(got_off, want_off)
    np.testing.assert_array_equal(got_keys, want_keys)
    np.testing.assert_array_equal(got_status, want_status)


def test_expand_flags_bad_ids(gpu):
    print("[lsa-cache] bad index / bucket ids, n_picked past the stride", flush=True)
    rng = np.random.default_rng(11)
    nidx, max_capacity = 4, 2048
    cache = LSABucketCache(nidx, max_capacity)
    sizes, members = _fill(rng, nidx, max_capacity, 1500)
    _upload(cache, sizes, members)
    B, stride = 6, 4
    ids = np.array([0, -1, nidx, 2, 3, 1])
    picked = rng.integers(0, cache.max_buckets, (B, stride))
    picked[3, 1] = cache.max_buckets  # one bad bucket id among good ones
    picked[4, 0] = -5
    n_picked = np.array([4, 4, 2, 4, 3, 9])  # 9 > stride
    pos = np.array([1400, 1400, 1400, 1400, 1400, 1400])
    got = _expand(cache, ids, picked, n_picked, pos, 64, 4, 16)
    want = _expected(sizes, members, ids, picked, n_picked, pos, 64, 4, 16, nidx, cache.max_buckets)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert list(got[2]) == [0, -6, -6, -6, -6, -6]


def test_expand_feeds_sparse_attention(gpu):
    # Device-built key lists into pkv_attend_sparse, 16q/2kv/512 fp32, against the oracle
    # attending the oracle-built lists.
    print("[lsa-cache] expand -> pkv_attend_sparse, 16q/2kv/512 fp32", flush=True)
    rng = np.random.default_rng(5)
    hq, hkv, d, bs = 16, 2, 512, 16
    B = 5
    ctx = np.array([600, 900, 1300, 2000, 2047])
    blocks = [(int(c) + bs) // bs for c in ctx]
    nb = sum(blocks) + 2
    stride_t = max(blocks) + 1
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride_t), np.int32)
    off = 0
    for s in range(B):
        tables[s, :blocks[s]] = perm[off:off + blocks[s]]
        off += blocks[s]
    kv = hkv * d
    k = rng.standard_normal(nb * bs * kv, dtype=np.float32)
    v = rng.standard_normal(nb * bs * kv, dtype=np.float32)
    q = rng.standard_normal((B, hq, d), dtype=np.float32)
    nidx = B
    cache = LSABucketCache(nidx, 2048)
    sizes, members = _fill(rng, nidx, 2048, 1)
    for s in range(B):  # members are positions below each sequence's context
        members[s] = rng.integers(0, int(ctx[s]) + 1, members[s].shape)
    _upload(cache, sizes, members)
    top_k, sink, window = 64, 4, 16
    ids = np.arange(B)
    picked = np.stack([rng.choice(cache.max_buckets, 4, replace=False) for _ in range(B)])
    n_picked = np.full(B, 4)
    dkeys, doff, dstatus = cache.expand(*[hip.DeviceArray.from_numpy(np.ascontiguousarray(a, np.int32))
                                          for a in (ids, picked, n_picked, ctx)],
                                        top_k, sink, window)
    assert np.all(dstatus.numpy() == 0)
    max_keys = LSABucketCache.max_keys(top_k, sink, window)
    p = make_params(LayerSpec(hq, hkv, d, window=0, kv_dtype=F32), bs, nb, 0.0625)
    ws_bytes = lib.load().pkv_sparse_workspace_size(ctypes.byref(p), B, max_keys)
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    dq, dk, dv, dt = (hip.DeviceArray.from_numpy(a) for a in (q, k, v, tables))
    out = hip.DeviceArray((B, hq, d), np.float32)
    lib.call("pkv_attend_sparse", None, ctypes.byref(p), dq.ptr, dk.ptr, dv.ptr, dt.ptr,
             stride_t, dkeys.ptr, doff.ptr, max_keys, B, out.ptr, ws.ptr, ws.nbytes)
    want_keys, want_off, _ = _expected(sizes, members, ids, picked, n_picked, ctx, top_k, sink,
                                       window, nidx, cache.max_buckets)
    ref = O.attend_sparse(q, k, v, tables, want_keys, want_off, hq, hkv, d, bs, scale=0.0625)
    exact = O.attend_sparse_f64(q, k, v, tables, want_keys, want_off, hq, hkv, d, bs,
                                scale=0.0625)
    parity.check(out.numpy(), ref, exact, what="expand->sparse")


def test_rollback_matches_oracle(gpu):
    print("[lsa-cache] rollback_to / reset, entries in order", flush=True)
    rng = np.random.default_rng(9)
    nidx, max_capacity = 12, 4096
    cache = LSABucketCache(nidx, max_capacity)
    maxb = cache.max_buckets
    closed = rng.integers(0, 9, nidx).astype(np.int32)  # 4096 / 512 = 8 blocks at most
    closed = np.minimum(closed, 8)
    total = (closed * 512 + rng.integers(0, 512, nidx)).astype(np.int32)
    sizes = rng.integers(1, CAP + 1, (nidx, maxb)).astype(np.int32)
    cache.sizes.upload_at(0, sizes)
    cache.closed_blocks.upload_at(0, closed)
    cache.total_tokens.upload_at(0, total)
    # entries: repeats, targets <= 0, past capacity, within a block, across several blocks,
    # and ids out of range (skipped)
    ids = np.array([0, 1, 2, 3, 3, 4, 5, 6, 7, 8, 9, 10, 11, -1, nidx, 5], np.int32)
    targets = np.array([510, 512, 0, 3000, 1000, -4, 9999, 1, 1024, 1023, 513, 4096, 2049, 7, 7,
                        100], np.int32)
    cache.rollback_to(hip.DeviceArray.from_numpy(ids), hip.DeviceArray.from_numpy(targets))
    states = []
    for i in range(nidx):
        st = O.LsaIndexState(max_capacity)
        st.closed_blocks[0], st.total_tokens[0] = closed[i], total[i]
        st.sizes[:] = sizes[i]
        states.append(st)
    for i, t in zip(ids, targets):
        if 0 <= i < nidx:
            states[i].rollback_to(int(t))
    np.testing.assert_array_equal(cache.closed_blocks.numpy(), [s.closed_blocks[0] for s in states])
    np.testing.assert_array_equal(cache.total_tokens.numpy(), [s.total_tokens[0] for s in states])
    np.testing.assert_array_equal(cache.sizes.numpy(), np.stack([s.sizes for s in states]))


def test_expand_reference_known_answer(gpu):
    """test_lsa_reference.mojo:130-184 through pkv_lsa_expand: position-mode buckets of 16
    tokens (bucket b = tokens 16b .. 16b + 15), picked [0, 2], position 63, top_k 10, sinks
    2, window 4 -> [2 .. 11, 60, 61, 62, 63, 0, 1]."""
    print("[lsa-cache] reference known answer", flush=True)
    cache = LSABucketCache(1, 512)
    sizes = np.zeros((1, cache.max_buckets), np.int32)
    members = np.zeros((1, cache.max_buckets, CAP), np.int32)
    for b in range(4):
        sizes[0, b] = 16
        members[0, b, :16] = np.arange(16 * b, 16 * b + 16)
    _upload(cache, sizes, members)
    keys, off, status = _expand(cache, np.array([0]), np.array([[0, 2]]), np.array([2]),
                                np.array([63]), 10, 2, 4)
    assert keys.tolist() == list(range(2, 12)) + [60, 61, 62, 63, 0, 1]
    assert off.tolist() == [0, 16] and status.tolist() == [lib.PKV_SEQ_OK]
