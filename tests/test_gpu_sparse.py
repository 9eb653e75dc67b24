"""GPU parity of LSA sparse paged attention (pkv_attend_sparse, lsa_core.mojo:630-680)
against the oracle's restatement, on key lists built by lsa_expand_buckets
(lsa_core.mojo:573-604) over the real global-layer geometry (16 q / 2 kv heads,
head_dim 512) and the configs' 16/8/256. Tolerances as tests/parity.py."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, hip, lib, lsa_expand_buckets
from pkv.engine import make_params
from tests import parity

pytestmark = pytest.mark.gpu


def _case(rng, B, ctx, hkv, d, kv_dtype):
    bs = 16
    kvs = hkv * d
    blocks = [(int(c) + bs) // bs for c in ctx]
    nb = sum(blocks) + 4
    stride = max(blocks) + 1
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride), np.int32)
    off = 0
    for s in range(B):
        tables[s, :blocks[s]] = perm[off:off + blocks[s]]
        off += blocks[s]
    k = rng.standard_normal(nb * bs * kvs, dtype=np.float32)
    v = rng.standard_normal(nb * bs * kvs, dtype=np.float32)
    if kv_dtype == BF16:
        k, v = O.to_bf16(k), O.to_bf16(v)
    return bs, nb, stride, tables, k, v


def _lists(rng, ctx, top_k, sinks, window):
    keys, off = [], [0]
    for pos in ctx:
        pos = int(pos)
        nb, cap = 16, 64
        sizes = np.minimum(rng.integers(0, cap + 1, nb), pos + 1)
        members = np.zeros((nb, cap), np.int64)
        for b in range(nb):
            members[b, :sizes[b]] = rng.choice(pos + 1, sizes[b], replace=False)
        picked = rng.choice(nb, 4, replace=False)
        sel = lsa_expand_buckets(picked, sizes, members, pos, top_k, sinks, window)
        keys.append(sel)
        off.append(off[-1] + sel.size)
    return np.concatenate(keys).astype(np.int32), np.asarray(off, np.int32)


def _run(p, q, k, v, tables, keys, off, max_keys, B, hq, d):
    ws_bytes = lib.load().pkv_sparse_workspace_size(ctypes.byref(p), B, max_keys)
    assert ws_bytes > 0
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    dq, dk, dv = hip.DeviceArray.from_numpy(q), hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    dt = hip.DeviceArray.from_numpy(tables)
    dkeys = hip.DeviceArray.from_numpy(keys if keys.size else np.zeros(1, np.int32))
    doff = hip.DeviceArray.from_numpy(off)
    out = hip.DeviceArray((B, hq, d), np.float32)
    lib.call("pkv_attend_sparse", None, ctypes.byref(p), dq.ptr, dk.ptr, dv.ptr, dt.ptr,
             tables.shape[1], dkeys.ptr, doff.ptr, max_keys, B, out.ptr, ws.ptr, ws.nbytes)
    return out.numpy()


@pytest.mark.parametrize("geom,kv_dtype,top_k,window", [
    ((16, 2, 512), F32, 64, 16),     # the model's global layers, LSA's small window
    ((16, 2, 512), BF16, 128, 256),
    ((16, 8, 256), F32, 512, 1024),  # lists longer than one 256-key chunk (merge path)
    ((16, 2, 256), F32, 256, 128),   # 8 rows per kv head at head_dim 256: the fp64 MFMA kernel
], ids=["g512-f32", "g512-bf16", "s256-long", "g256-f32-mfma"])
def test_sparse_lists_match_oracle(gpu, geom, kv_dtype, top_k, window):
    print(f"[sparse] {geom} {kv_dtype} top_k={top_k} window={window}", flush=True)
    rng = np.random.default_rng(top_k + window)
    hq, hkv, d = geom
    B = 6
    ctx = np.array([0, 5, 700, 1500, 2600, 4000])
    bs, nb, stride, tables, k, v = _case(rng, B, ctx, hkv, d, kv_dtype)
    keys, off = _lists(rng, ctx, top_k, 4, window)
    q = rng.standard_normal((B, hq, d), dtype=np.float32)
    p = make_params(LayerSpec(hq, hkv, d, window=0, kv_dtype=kv_dtype), bs, nb, 0.0625)
    max_keys = int(np.diff(off).max())
    got = _run(p, q, k, v, tables, keys, off, max_keys, B, hq, d)
    ref = O.attend_sparse(q, k, v, tables, keys, off, hq, hkv, d, bs, scale=0.0625,
                          nthreads=O.max_threads(), par=1)
    exact = None
    if kv_dtype == F32:
        exact = O.attend_sparse_f64(q, k, v, tables, keys, off, hq, hkv, d, bs, scale=0.0625)
    parity.check(got, ref, exact, bf16=kv_dtype == BF16, what="sparse")


@pytest.mark.parametrize("d", [512, 256], ids=["d512", "d256-mfma"])
def test_sparse_empty_bad_and_overlong_lists(gpu, d):
    # An empty list gives zeros; a key past the table or a list longer than max_keys NaN.
    print(f"[sparse] empty / bad key / overlong, head_dim {d}", flush=True)
    rng = np.random.default_rng(3)
    hq, hkv = 16, 2
    B = 4
    ctx = np.array([100, 100, 100, 100])
    bs, nb, stride, tables, k, v = _case(rng, B, ctx, hkv, d, F32)
    lists = [np.arange(0, 50), np.array([], np.int64), np.array([3, 7, stride * bs + 5]),
             np.arange(0, 101)]
    keys = np.concatenate(lists).astype(np.int32)
    off = np.concatenate([[0], np.cumsum([x.size for x in lists])]).astype(np.int32)
    q = rng.standard_normal((B, hq, d), dtype=np.float32)
    p = make_params(LayerSpec(hq, hkv, d), bs, nb, 1.0)
    got = _run(p, q, k, v, tables, keys, off, 60, B, hq, d)
    ref0 = O.attend_sparse(q[:1], k, v, tables[:1], keys[:50], off[:2], hq, hkv, d, bs)
    parity.check(got[:1], ref0, O.attend_sparse_f64(q[:1], k, v, tables[:1], keys[:50], off[:2],
                                                    hq, hkv, d, bs), what="list 0")
    assert np.all(got[1] == 0.0)
    assert np.all(np.isnan(got[2])) and np.all(np.isnan(got[3]))
