"""pkv_attend_noalloc (no workspace argument; partials in the library's 64 MiB device
scratch) against pkv_attend with a caller workspace, through the C ABI. Two decode calls in
a row, the second with a smaller batch and shorter contexts (the scratch keeps the first
call's contents, which must not leak into the second): there the scratch holds partials
for as many workgroups as pkv_attend's workspace, so both take the same key split and the
outputs are bit-identical. Then a 4-query verify on the fp64 MFMA kernel, whose rows need
more scratch per workgroup: it is held to the parity rule against pkv_attend's output and
the oracle (the two may split the keys differently). A call whose partials cannot fit the
scratch is refused with PKV_ERR_WORKSPACE before anything is launched. A bf16-pool verify
runs the bf16 MFMA kernel (fp32 partials) through the scratch. Last, the entry point under
HIP graph capture (relaxed mode) after one eager call: the graph replayed three times, with
new queries written eagerly between replays, against pkv_attend."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, PagedKVCache, hip, lib
from pkv.engine import make_params
from tests import parity

pytestmark = pytest.mark.gpu

BS = 16


def _noalloc(cache, q, pos, q_len, out, batch, max_pos):
    p = cache.params[0]
    lib.call("pkv_attend_noalloc", None, ctypes.byref(p), q.ptr, cache.k_pools[0].ptr,
             cache.v_pools[0].ptr, cache.tables.ptr, cache.table_stride,
             cache._ints(pos, cache._i32_a, batch), q_len, batch, max_pos, out.ptr)


def _setup(rng, B, ctx, max_q_len):
    spec = LayerSpec(16, 8, 256, window=0, kv_dtype=F32)
    stride = int((ctx.max() + max_q_len + BS - 1) // BS) + 1
    lens = ((ctx + max_q_len + BS - 1) // BS).astype(np.int32)
    nb = int(lens.sum()) + 4
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride), np.int32)
    o = 0
    for s in range(B):
        tables[s, :lens[s]] = perm[o:o + lens[s]]
        o += lens[s]
    cache = PagedKVCache([spec], block_size=BS, num_blocks=nb, max_seqs=B,
                         max_blocks_per_seq=stride, max_q_len=max_q_len,
                         max_pos=stride * BS - 1, scale=0.0625)
    cache.tables.upload(tables)
    cache.table_lens.upload(lens)
    kp = rng.standard_normal(cache.k_pools[0].shape, dtype=np.float32)
    vp = rng.standard_normal(cache.v_pools[0].shape, dtype=np.float32)
    cache.k_pools[0].upload(kp)
    cache.v_pools[0].upload(vp)
    return cache, tables, lens, kp.reshape(-1), vp.reshape(-1)


def _pair(cache, q, pos, q_len, batch, what, bitwise=True):
    print(f"[no_alloc] {what}: batch {batch}, q_len {q_len}", flush=True)
    dq = hip.DeviceArray.from_numpy(q)
    shape = (batch, q_len, 16, 256)
    out_ws = hip.DeviceArray(shape, np.float32)
    out_na = hip.DeviceArray(shape, np.float32)
    max_pos = int(pos.max()) + q_len - 1
    cache.attend(0, dq, pos, q_len, out_ws, batch=batch, max_pos=max_pos)
    _noalloc(cache, dq, pos, q_len, out_na, batch, max_pos)
    a, b = out_ws.numpy(), out_na.numpy()
    if bitwise:
        assert np.array_equal(a, b), f"{what}: outputs differ from pkv_attend's"
    else:  # both near-exact attention: within the float64 bound of each other
        assert np.all(np.isfinite(b)) and O.max_rel_err(b, a) <= parity.TOL_EXACT, what
    return b


def test_noalloc_matches_attend_twice_then_verify(gpu):
    rng = np.random.default_rng(77)
    B = 32
    ctx = rng.integers(100, 3000, B).astype(np.int32)
    cache, tables, lens, kp, vp = _setup(rng, B, ctx, 4)
    # call 1: 32 decode queries
    q1 = rng.standard_normal((B, 1, 16, 256), dtype=np.float32)
    got1 = _pair(cache, q1, ctx, 1, B, "call 1")
    ref = O.attend(q1, kp, vp, tables, lens, ctx, 1, 16, 8, 256, BS, 0, scale=0.0625,
                   nthreads=O.max_threads(), par=1)
    exact = O.attend_f64(q1, kp, vp, tables, ctx, 1, 16, 8, 256, BS, 0, scale=0.0625)
    parity.check(got1, ref, exact, what="no-alloc call 1")
    # call 2: a smaller input -- 5 sequences, shorter contexts
    pos2 = (ctx[:5] // 3).astype(np.int32)
    q2 = rng.standard_normal((5, 1, 16, 256), dtype=np.float32)
    got2 = _pair(cache, q2, pos2, 1, 5, "call 2")
    ref = O.attend(q2, kp, vp, tables[:5], lens[:5], pos2, 1, 16, 8, 256, BS, 0, scale=0.0625)
    exact = O.attend_f64(q2, kp, vp, tables[:5], pos2, 1, 16, 8, 256, BS, 0, scale=0.0625)
    parity.check(got2, ref, exact, what="no-alloc call 2")
    # call 3: a 4-query verify (8 rows per kv head: the fp64 MFMA kernel)
    q3 = rng.standard_normal((16, 4, 16, 256), dtype=np.float32)
    got3 = _pair(cache, q3, ctx[:16], 4, 16, "call 3 (verify)", bitwise=False)
    ref = O.attend(q3, kp, vp, tables[:16], lens[:16], ctx[:16], 4, 16, 8, 256, BS, 0,
                   scale=0.0625, nthreads=O.max_threads(), par=1)
    exact = O.attend_f64(q3, kp, vp, tables[:16], ctx[:16], 4, 16, 8, 256, BS, 0, scale=0.0625)
    parity.check(got3, ref, exact, what="no-alloc call 3")
    cache.free()


def test_noalloc_refuses_partials_beyond_the_scratch(gpu):
    # 16 q heads at head_dim 512 with 16 queries: 256 rows of 514 doubles per slot, ~1 MiB,
    # so 64 sequences need more than the 64 MiB scratch holds.
    print("[no_alloc] oversized call is refused", flush=True)
    p = make_params(LayerSpec(16, 2, 512), BS, 64)
    buf = hip.DeviceArray((1024,), np.uint8, zero=True)
    rc = lib.load().pkv_attend_noalloc(None, ctypes.byref(p), buf.ptr, buf.ptr, buf.ptr,
                                       buf.ptr, 4, buf.ptr, 16, 64, 63, buf.ptr)
    assert rc == lib.PKV_ERR_WORKSPACE, rc
    buf.free()


def test_noalloc_bf16_verify(gpu):
    """bf16 pools, 4 queries at G = 2 (8 rows per kv head: the bf16 MFMA kernel, whose
    partials are fp32): pkv_attend_noalloc against pkv_attend with a workspace (within the
    float64 bound of each other) and both against the oracle on the same bf16 values."""
    print("[no_alloc] bf16 verify", flush=True)
    rng = np.random.default_rng(55)
    B, q_len, hq, hkv, d = 16, 4, 16, 8, 256
    ctx = rng.integers(100, 3000, B).astype(np.int32)
    blocks = (ctx + q_len + BS - 1) // BS
    nb = int(blocks.sum()) + 4
    stride = int(blocks.max()) + 1
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride), np.int32)
    o = 0
    for s in range(B):
        tables[s, :blocks[s]] = perm[o:o + blocks[s]]
        o += blocks[s]
    k = O.to_bf16(rng.standard_normal(nb * BS * hkv * d, dtype=np.float32))
    v = O.to_bf16(rng.standard_normal(nb * BS * hkv * d, dtype=np.float32))
    q = rng.standard_normal((B, q_len, hq, d), dtype=np.float32)
    p = make_params(LayerSpec(hq, hkv, d, 0, BF16), BS, nb, 0.0625)
    max_pos = int(ctx.max()) + q_len - 1
    dk, dv = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    dt, dq, dpos = (hip.DeviceArray.from_numpy(x) for x in (tables, q, ctx))
    out_ws = hip.DeviceArray(q.shape, np.float32)
    out_na = hip.DeviceArray(q.shape, np.float32)
    ws_bytes = lib.load().pkv_workspace_size(ctypes.byref(p), B, q_len, max_pos)
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    lib.call("pkv_attend", None, ctypes.byref(p), dq.ptr, dk.ptr, dv.ptr, dt.ptr, stride,
             dpos.ptr, q_len, B, max_pos, out_ws.ptr, ws.ptr, ws.nbytes)
    lib.call("pkv_attend_noalloc", None, ctypes.byref(p), dq.ptr, dk.ptr, dv.ptr, dt.ptr, stride,
             dpos.ptr, q_len, B, max_pos, out_na.ptr)
    a, b = out_ws.numpy(), out_na.numpy()
    assert np.all(np.isfinite(b)) and O.max_rel_err(b, a) <= parity.TOL_EXACT
    lens = blocks.astype(np.int32)
    ref = O.attend(q, k, v, tables, lens, ctx, q_len, hq, hkv, d, BS, 0, scale=0.0625,
                   nthreads=O.max_threads(), par=1)
    parity.check(b, ref, bf16=True, what="no-alloc bf16 verify")
    for x in (dk, dv, dt, dq, dpos, out_ws, out_na, ws):
        x.free()


def _graph_api():
    h = hip._lib()
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    for name, args in (("hipStreamBeginCapture", [vp, i32]),
                       ("hipStreamEndCapture", [vp, ctypes.POINTER(vp)]),
                       ("hipGraphInstantiate", [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]),
                       ("hipGraphExecDestroy", [vp]),
                       ("hipGraphDestroy", [vp])):
        fn = getattr(h, name)
        fn.argtypes = args
        fn.restype = i32
    return h


@pytest.mark.parametrize("q_len", [1, 4], ids=["decode", "verify-mfma"])
def test_noalloc_under_graph_capture(gpu, q_len):
    """One eager call (the scratch's address and the kernels' launch set-up are looked up on
    a device's first call), then pkv_attend_noalloc captured on a stream in relaxed mode,
    instantiated and replayed three times; before each replay new queries are copied into
    the captured input eagerly, and each replay's output is checked against pkv_attend on
    the same inputs (bit-identical for decode, where both take the same key split; the
    parity rule for the verify)."""
    print(f"[no_alloc] graph capture q_len={q_len}", flush=True)
    rng = np.random.default_rng(91 + q_len)
    B = 16
    ctx = rng.integers(100, 2000, B).astype(np.int32)
    cache, tables, lens, kp, vp = _setup(rng, B, ctx, q_len)
    h = _graph_api()
    stream = hip.Stream()
    p = cache.params[0]
    shape = (B, q_len, 16, 256)
    dq = hip.DeviceArray(shape, np.float32)
    dpos = hip.DeviceArray.from_numpy(ctx)
    out_g = hip.DeviceArray(shape, np.float32)
    out_ref = hip.DeviceArray(shape, np.float32)
    max_pos = int(ctx.max()) + q_len - 1

    def call():
        return lib.load().pkv_attend_noalloc(
            ctypes.c_void_p(stream.handle), ctypes.byref(p), ctypes.c_void_p(dq.ptr),
            ctypes.c_void_p(cache.k_pools[0].ptr), ctypes.c_void_p(cache.v_pools[0].ptr),
            ctypes.c_void_p(cache.tables.ptr), cache.table_stride, ctypes.c_void_p(dpos.ptr),
            q_len, B, max_pos, ctypes.c_void_p(out_g.ptr))

    dq.upload(rng.standard_normal(shape, dtype=np.float32))
    assert call() == 0, lib.load().pkv_last_error().decode()  # eager warm-up call
    stream.synchronize()
    graph, gexec = ctypes.c_void_p(), ctypes.c_void_p()
    hip.check(h.hipStreamBeginCapture(ctypes.c_void_p(stream.handle), 2), "hipStreamBeginCapture")
    rc = call()
    hip.check(h.hipStreamEndCapture(ctypes.c_void_p(stream.handle), ctypes.byref(graph)),
              "hipStreamEndCapture")
    assert rc == 0, lib.load().pkv_last_error().decode()
    hip.check(h.hipGraphInstantiate(ctypes.byref(gexec), graph, None, None, 0),
              "hipGraphInstantiate")
    for rep in range(3):
        q = rng.standard_normal(shape, dtype=np.float32)
        dq.upload(q)  # eager work between replays
        out_g.fill_bytes_(0xFF)
        hip.check(h.hipGraphLaunch(gexec, ctypes.c_void_p(stream.handle)), "hipGraphLaunch")
        stream.synchronize()
        got = out_g.numpy()
        cache.attend(0, dq, ctx, q_len, out_ref, batch=B, max_pos=max_pos)
        ref_ws = out_ref.numpy()
        if q_len == 1:
            assert np.array_equal(got, ref_ws), f"replay {rep}: differs from pkv_attend"
        else:
            assert np.all(np.isfinite(got)) and O.max_rel_err(got, ref_ws) <= parity.TOL_EXACT
        ref = O.attend(q, kp, vp, tables, lens, ctx, q_len, 16, 8, 256, BS, 0, scale=0.0625,
                       nthreads=O.max_threads(), par=1)
        exact = O.attend_f64(q, kp, vp, tables, ctx, q_len, 16, 8, 256, BS, 0, scale=0.0625)
        parity.check(got, ref, exact, what=f"graph replay {rep}")
    h.hipGraphExecDestroy(gexec)
    h.hipGraphDestroy(graph)
    stream.destroy()
    cache.free()
