"""GPU parity of K2 (split-K paged attention) against the oracle's restatement of
paged_attention_layer (attention.mojo:240-294), on the reference's own test fixtures
(test_attention.mojo) and on seeded N(0,1) data. Tolerances (tests/parity.py): max
|x-ref|/(|ref|+1e-3) <= 1e-4 for fp32 pools (and <= 1e-5 against float64 attention),
<= 2e-2 for bf16 pools (oracle on the upcast values)."""
import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, hip, lib, paged_attention_layer
from pkv.engine import make_params
from tests import parity
from tests.refcase import BLOCK_SIZE, CAPACITY, NUM_BLOCKS, Fixture

pytestmark = pytest.mark.gpu


class DevFixture:
    """The reference Fixture uploaded to the device."""

    def __init__(self, fx: Fixture, kv_dtype=F32):
        self.fx = fx
        self.kv_dtype = kv_dtype
        if kv_dtype == BF16:
            self.k_host, self.v_host = O.to_bf16(fx.k_pool), O.to_bf16(fx.v_pool)
        else:
            self.k_host, self.v_host = fx.k_pool, fx.v_pool
        self.k = hip.DeviceArray.from_numpy(self.k_host)
        self.v = hip.DeviceArray.from_numpy(self.v_host)
        self.table = hip.DeviceArray.from_numpy(fx.table.astype(np.int32))
        self.q = hip.DeviceArray.from_numpy(fx.q)
        self.out = hip.DeviceArray((fx.heads * fx.head_dim + 64,), np.float32)

    def refresh(self):
        self.k.upload(O.to_bf16(self.fx.k_pool) if self.kv_dtype == BF16 else self.fx.k_pool)
        self.v.upload(O.to_bf16(self.fx.v_pool) if self.kv_dtype == BF16 else self.fx.v_pool)

    def run(self, pos, window):
        fx = self.fx
        canary = np.full(fx.heads * fx.head_dim + 64, -12345.678, np.float32)
        self.out.upload(canary)
        paged_attention_layer(self.q, self.k, self.v, self.table, BLOCK_SIZE, pos, fx.heads,
                              fx.kv_heads, fx.head_dim, window, self.out, num_blocks=NUM_BLOCKS,
                              kv_dtype=self.kv_dtype)
        o = self.out.numpy()
        assert np.all(o[fx.heads * fx.head_dim:] == np.float32(-12345.678)), "attn_out overflow"
        return o[: fx.heads * fx.head_dim]

    def oracle(self, pos, window):
        return O.paged_attention_layer(self.fx.q, self.k_host, self.v_host, self.fx.table,
                                       BLOCK_SIZE, pos, self.fx.heads, self.fx.kv_heads,
                                       self.fx.head_dim, window)

    def exact(self, pos, window):
        return O.attention_f64(self.fx.q, self.k_host, self.v_host, self.fx.table, BLOCK_SIZE,
                               pos, O.window_start(pos, window), self.fx.heads,
                               self.fx.kv_heads, self.fx.head_dim)

    def check(self, pos, window):
        out = self.run(pos, window)
        bf16 = self.kv_dtype == BF16
        parity.check(out, self.oracle(pos, window), None if bf16 else self.exact(pos, window),
                     bf16=bf16, what=f"pos={pos} window={window}")
        return out


@pytest.mark.parametrize("geom", [(16, 2, 512), (16, 8, 256), (8, 8, 64), (12, 4, 256)],
                         ids=["global", "sliding", "ratio1", "ratio3"])
@pytest.mark.parametrize("window", [0, 1024])
def test_fixture_positions_match_oracle(gpu, geom, window):
    print(f"[attend] geom={geom} window={window}", flush=True)
    d = DevFixture(Fixture(*geom, seed=42, k_scale=0.25))
    for p in [0, 1, 15, 16, 17, 63, 64, 99, 255, 256, 257, 777, 1023, 1024, 1500, CAPACITY - 1]:
        d.check(p, window)


def test_short_windows_and_f64(gpu):
    print("[attend] short windows", flush=True)
    d = DevFixture(Fixture(16, 8, 256, seed=99, k_scale=0.25))
    for p in [1024, 1025, 1500, 2047, CAPACITY - 1]:
        for w in [1, 7, 1024]:
            d.check(p, w)
        # the reference's own check: windowed result vs float64, < 1e-4 (:311-321)
        assert O.max_rel_err(d.run(p, 1024), d.fx.run_reference(p, p - 1023)) < 1e-4


def test_single_key_is_value_row(gpu):
    d = DevFixture(Fixture(16, 8, 256, seed=4, k_scale=1.0))
    out = d.run(777, 1)
    r = d.fx.row_of(777)
    for h in range(16):
        g = h // 2
        np.testing.assert_array_equal(out[h * 256:(h + 1) * 256],
                                      d.fx.v_pool[r + g * 256:r + (g + 1) * 256])


def test_window_edges_planted(gpu):
    # test_attention.mojo:324-365 and :440-497 on the GPU.
    print("[attend] planted keys", flush=True)
    fx = Fixture(16, 8, 256, seed=3, k_scale=0.01)
    d = DevFixture(fx)
    pos = 2000
    fx.plant(pos - 1024)
    d.refresh()
    assert np.all(np.abs(d.run(pos, 1024)) < 10.0)
    fx.plant(pos - 1023)
    d.refresh()
    assert np.all(d.run(pos, 1024) > 900.0)
    fx2 = Fixture(16, 8, 256, seed=21, k_scale=0.01)
    pos2 = 1024 + 16 * 3 + 1023
    start = O.window_start(pos2, 1024)
    fx2.plant(start - 1)
    d2 = DevFixture(fx2)
    assert np.all(np.abs(d2.run(pos2, 1024)) < 10.0)
    fx2.plant(start)
    d2.refresh()
    assert np.all(d2.run(pos2, 1024) > 900.0)
    fx3 = Fixture(16, 8, 256, seed=22, k_scale=0.01)
    fx3.plant(1777)
    assert np.all(DevFixture(fx3).run(1777, 1024) > 900.0)


def test_large_scores_finite(gpu):
    d = DevFixture(Fixture(16, 2, 512, seed=11, k_scale=4.0))
    for p in [0, 300, CAPACITY - 1]:
        out = d.check(p, 0)
        assert np.all(np.isfinite(out)) and np.all(np.abs(out) < 1e30)


@pytest.mark.parametrize("geom", [(16, 8, 256), (16, 2, 512)])
def test_bf16_pools(gpu, geom):
    print(f"[attend] bf16 {geom}", flush=True)
    d = DevFixture(Fixture(*geom, seed=5, k_scale=0.5), kv_dtype=BF16)
    for p in [0, 100, 1023, 2047, CAPACITY - 1]:
        d.check(p, 0)


def _batched_case(rng, B, q_len, ctx, hq, hkv, d, bs, window, kv_dtype, scale):
    kvs = hkv * d
    blocks_per = [(int(c) + q_len + bs - 1) // bs for c in ctx]
    nb = sum(blocks_per) + 8
    stride = max(blocks_per) + 2
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride), np.int32)
    lens = np.zeros(B, np.int32)
    off = 0
    for s in range(B):
        tables[s, :blocks_per[s]] = perm[off:off + blocks_per[s]]
        lens[s] = blocks_per[s]
        off += blocks_per[s]
    k = rng.standard_normal(nb * bs * kvs, dtype=np.float32)
    v = rng.standard_normal(nb * bs * kvs, dtype=np.float32)
    if kv_dtype == BF16:
        k, v = O.to_bf16(k), O.to_bf16(v)
    q = rng.standard_normal((B, q_len, hq, d), dtype=np.float32)
    pos = np.asarray(ctx, np.int32)
    ref = O.attend(q, k, v, tables, lens, pos, q_len, hq, hkv, d, bs, window, scale=scale,
                   nthreads=O.max_threads(), par=1)
    exact = None if kv_dtype == BF16 else O.attend_f64(q, k, v, tables, pos, q_len, hq, hkv, d,
                                                        bs, window, scale=scale)
    spec = LayerSpec(hq, hkv, d, window, kv_dtype)
    p = make_params(spec, bs, nb, scale)
    import ctypes
    max_pos = int(pos.max()) + q_len - 1
    ws_bytes = lib.load().pkv_workspace_size(ctypes.byref(p), B, q_len, max_pos)
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    dk, dv = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    dt, dq = hip.DeviceArray.from_numpy(tables), hip.DeviceArray.from_numpy(q)
    dpos = hip.DeviceArray.from_numpy(pos)
    out = hip.DeviceArray((B, q_len, hq, d), np.float32)
    for rep in range(2):  # the second call reuses the self-resetting chunk counters
        lib.call("pkv_attend", None, ctypes.byref(p), dq.ptr, dk.ptr, dv.ptr, dt.ptr, stride,
                 dpos.ptr, q_len, B, max_pos, out.ptr, ws.ptr, ws.nbytes)
        got = out.numpy()
        parity.check(got, ref, exact, bf16=kv_dtype == BF16, what=f"rep {rep}")
    return got


def test_single_sequence_over_many_pieces(gpu):
    # One kv head keeps the stream kernel's workgroups small, so up to 1024 of them split
    # 40,000 keys of one sequence: the merge then combines far more pieces than its
    # register-held first 32 and more than one per thread of its workgroup.
    print("[attend] one sequence, 40000 keys, 2q/1kv/256 fp32", flush=True)
    rng = np.random.default_rng(40000)
    _batched_case(rng, 1, 1, np.array([40000]), 2, 1, 256, 16, 0, F32, 0.0625)


@pytest.mark.parametrize("window", [0, 1024])
def test_batched_mixed_contexts(gpu, window):
    print(f"[attend] batched mixed window={window}", flush=True)
    rng = np.random.default_rng(7)
    ctx = rng.integers(128, 3000, 12)
    ctx[0], ctx[1] = 0, 255  # single key and exactly one chunk
    _batched_case(rng, 12, 1, ctx, 16, 8, 256, 16, window, F32, 0.0625)


@pytest.mark.parametrize("q_len", [2, 4, 8])
def test_verify_queries_causal(gpu, q_len):
    print(f"[attend] verify q_len={q_len}", flush=True)
    rng = np.random.default_rng(q_len)
    ctx = rng.integers(500, 2500, 6)
    _batched_case(rng, 6, q_len, ctx, 16, 8, 256, 16, 0, F32, 0.0625)


def test_verify_sliding_bf16(gpu):
    rng = np.random.default_rng(11)
    ctx = rng.integers(900, 2100, 5)
    _batched_case(rng, 5, 4, ctx, 16, 8, 256, 16, 1024, BF16, 0.0625)


@pytest.mark.parametrize("geom,q_len,window,kv_dtype", [
    ((16, 2, 512), 5, 0, F32),     # the model's global layers: 5 verify queries, 40 rows
    ((16, 2, 512), 5, 0, BF16),
    ((16, 8, 256), 9, 1024, F32),  # sliding: 9 queries (18 rows) in query groups
], ids=["g512-f32", "g512-bf16", "s256-q9"])
def test_verify_query_groups(gpu, geom, q_len, window, kv_dtype):
    print(f"[attend] verify query groups {geom} q_len={q_len}", flush=True)
    rng = np.random.default_rng(q_len + geom[2])
    ctx = rng.integers(300, 3000, 5)
    ctx[0] = 0
    _batched_case(rng, 5, q_len, ctx, *geom, 16, window, kv_dtype, 0.0625)


@pytest.mark.parametrize("hq,hkv,q_len,window", [
    (32, 16, 4, 0),     # 16 kv heads: two workgroup head groups
    (8, 8, 8, 0),       # G = 1: 8 queries per kv head
    (24, 8, 2, 0),      # G = 3: 6 rows (a partly filled row group)
    (16, 4, 2, 0),      # G = 4
    (16, 8, 3, 600),    # 6 rows with a window
], ids=["hkv16", "g1-q8", "g3-q2", "g4-q2", "q3-window"])
def test_verify_fp64_mfma_geometries(gpu, hq, hkv, q_len, window):
    # fp32 pools, head_dim 256, 5..8 query rows per kv head: stream_mfma_kernel
    print(f"[attend] fp64 MFMA verify {hq}q/{hkv}kv q_len={q_len} window={window}", flush=True)
    rng = np.random.default_rng(hq * 7 + hkv + q_len)
    ctx = rng.integers(100, 1800, 5)
    ctx[0] = 0
    _batched_case(rng, 5, q_len, ctx, hq, hkv, 256, 16, window, F32, 0.0625)


def test_verify_inactive_and_bad_table_mfma(gpu):
    # The contract paths of the fp64 MFMA verify kernel (16/8/256, 4 queries = 8 rows per
    # kv head): an inactive sequence gives zeros, a table entry outside the pool NaN, a
    # call past max_pos NaN; the other sequences stay finite.
    print("[attend] MFMA verify inactive / bad table", flush=True)
    import ctypes
    rng = np.random.default_rng(31)
    B, hq, hkv, d, bs, nb, stride, ql = 3, 16, 8, 256, 16, 64, 8, 4
    p = make_params(LayerSpec(hq, hkv, d), bs, nb, 0.0625)
    tables = rng.integers(0, nb, (B, stride)).astype(np.int32)
    tables[2, 3] = nb + 5  # out of the pool
    k = hip.DeviceArray.from_numpy(rng.standard_normal(nb * bs * hkv * d, dtype=np.float32))
    q = hip.DeviceArray.from_numpy(rng.standard_normal((B, ql, hq, d), dtype=np.float32))
    out = hip.DeviceArray((B, ql, hq, d), np.float32)
    ws_bytes = lib.load().pkv_workspace_size(ctypes.byref(p), B, ql, 127)
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    dtab = hip.DeviceArray.from_numpy(tables)
    dpos = hip.DeviceArray.from_numpy(np.array([40, -1, 60], np.int32))
    lib.call("pkv_attend", None, ctypes.byref(p), q.ptr, k.ptr, k.ptr, dtab.ptr, stride,
             dpos.ptr, ql, B, 127, out.ptr, ws.ptr, ws.nbytes)
    o = out.numpy()
    assert np.all(np.isfinite(o[0]))
    assert np.all(o[1] == 0.0)
    assert np.all(np.isnan(o[2]))
    dtab2 = hip.DeviceArray.from_numpy(np.clip(tables, 0, nb - 1))
    dpos2 = hip.DeviceArray.from_numpy(np.array([40, 125, 0], np.int32))  # 125 + 3 > 127
    lib.call("pkv_attend", None, ctypes.byref(p), q.ptr, k.ptr, k.ptr, dtab2.ptr, stride,
             dpos2.ptr, ql, B, 127, out.ptr, ws.ptr, ws.nbytes)
    o = out.numpy()
    assert np.all(np.isnan(o[1])) and np.all(np.isfinite(o[0])) and np.all(np.isfinite(o[2]))


@pytest.mark.parametrize("hq,hkv,q_len,bs,window", [
    (16, 8, 4, 16, 0),     # config 5's shape with bf16 pools: 8 rows per kv head
    (16, 8, 4, 16, 1024),  # the sliding layers' window
    (16, 8, 3, 16, 0),     # 6 rows: two columns of each half unused
    (16, 16, 8, 16, 0),    # G = 1, 8 queries; 16 kv heads: two workgroup head groups
    (16, 4, 2, 16, 0),     # G = 4
    (16, 2, 1, 16, 0),     # G = 8 decode at head_dim 256
    (16, 8, 4, 2, 0),      # smallest block size the kernel takes (a copy pair in one block)
    (16, 8, 4, 64, 33),    # large blocks, an odd window
], ids=["cfg5", "window", "rows6", "g1-q8", "g4", "g8", "bs2", "bs64-w33"])
def test_verify_bf16_mfma(gpu, hq, hkv, q_len, bs, window):
    """bf16 pools with 5..8 query rows per kv head (stream_bf16_mfma_kernel: QK^T and PV on
    the bf16 matrix cores with Q and P split into hi + lo bf16 parts): mixed contexts from a
    single key to multi-piece sequences, odd and even first and last keys (the kernel's copy
    pairs start on even positions), against the oracle on the same bf16 values (2e-2)."""
    print(f"[attend] bf16 mfma {hq}q/{hkv}kv q_len {q_len} bs {bs} window {window}", flush=True)
    rng = np.random.default_rng(hq * 100 + hkv * 10 + q_len + bs + window)
    ctx = np.concatenate([[0, 1, 2, 3, 16, 17, 31], rng.integers(40, 5000, 9)])
    _batched_case(rng, ctx.size, q_len, ctx, hq, hkv, 256, bs, window, BF16, 0.0625)


@pytest.mark.parametrize("q_len", [1, 4], ids=["decode-vector", "verify-mfma"])
def test_batch_4096_large_lds(gpu, q_len):
    """The largest batch pkv_attend takes: the stream kernels keep 5 ints per sequence in
    LDS, ~80 KiB at 4096, above the 64 KiB a kernel gets without opting in (the vector
    kernel for decode, interleaved; the fp64 MFMA kernel, 8 rows per kv head, for 4 queries,
    in its one-wave-per-kv-head form, since the interleaved form's exchange area no longer
    fits)."""
    print(f"[attend] batch 4096, q_len {q_len}", flush=True)
    rng = np.random.default_rng(4096 + q_len)
    ctx = rng.integers(1, 48, 4096)
    _batched_case(rng, 4096, q_len, ctx, 2, 1, 256, 16, 0, F32, 0.0625)


def test_bf16_verify_batch_512(gpu):
    """bf16 pools, 8 rows per kv head, 512 sequences: the interleaved bf16 MFMA kernel's
    exchange area no longer fits beside the per-sequence ints, so the launch takes the
    one-wave-per-kv-head form of the same kernel."""
    print("[attend] bf16 verify, batch 512", flush=True)
    rng = np.random.default_rng(512)
    ctx = rng.integers(1, 300, 512)
    _batched_case(rng, 512, 4, ctx, 16, 8, 256, 16, 0, BF16, 0.0625)


def test_gqa8_d512(gpu):
    rng = np.random.default_rng(12)
    ctx = rng.integers(1, 4000, 4)
    _batched_case(rng, 4, 1, ctx, 16, 2, 512, 16, 0, F32, 1.0)


def test_inactive_sequence_gives_zeros_and_bad_table_gives_nan(gpu):
    print("[attend] inactive / bad table", flush=True)
    import ctypes
    rng = np.random.default_rng(3)
    B, hq, hkv, d, bs, nb, stride = 3, 16, 8, 256, 16, 64, 8
    spec = LayerSpec(hq, hkv, d)
    p = make_params(spec, bs, nb, 1.0)
    tables = rng.integers(0, nb, (B, stride)).astype(np.int32)
    tables[2, 3] = nb + 5  # out of the pool
    k = hip.DeviceArray((nb * bs * hkv * d,), np.float32, zero=True)
    q = hip.DeviceArray.from_numpy(rng.standard_normal((B, 1, hq, d), dtype=np.float32))
    pos = np.array([40, -1, 60], np.int32)
    out = hip.DeviceArray((B, 1, hq, d), np.float32)
    ws_bytes = lib.load().pkv_workspace_size(ctypes.byref(p), B, 1, 127)
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    # device arguments stay referenced until the results are read back
    dtab, dpos = hip.DeviceArray.from_numpy(tables), hip.DeviceArray.from_numpy(pos)
    lib.call("pkv_attend", None, ctypes.byref(p), q.ptr, k.ptr, k.ptr, dtab.ptr, stride,
             dpos.ptr, 1, B, 127, out.ptr, ws.ptr, ws.nbytes)
    o = out.numpy()
    np.testing.assert_allclose(o[0], 0.0, atol=0)  # zero V rows
    assert np.all(o[1] == 0.0)
    assert np.all(np.isnan(o[2]))
    # pos beyond max_pos -> NaN, never an out-of-grid read
    pos2 = np.array([40, 200, 0], np.int32)
    dtab2 = hip.DeviceArray.from_numpy(np.clip(tables, 0, nb - 1))
    dpos2 = hip.DeviceArray.from_numpy(pos2)
    lib.call("pkv_attend", None, ctypes.byref(p), q.ptr, k.ptr, k.ptr, dtab2.ptr, stride,
             dpos2.ptr, 1, B, 127, out.ptr, ws.ptr, ws.nbytes)
    o = out.numpy()
    assert np.all(np.isnan(o[1])) and np.all(np.isfinite(o[0])) and np.all(np.isfinite(o[2]))
    # beyond max_pos but inside the table stride -> NaN as well (the grid is sized by it)
    stride3 = 16
    dtab3 = hip.DeviceArray.from_numpy(rng.integers(0, nb, (B, stride3)).astype(np.int32))
    lib.call("pkv_attend", None, ctypes.byref(p), q.ptr, k.ptr, k.ptr, dtab3.ptr, stride3,
             dpos2.ptr, 1, B, 127, out.ptr, ws.ptr, ws.nbytes)
    o = out.numpy()
    assert np.all(np.isnan(o[1])) and np.all(np.isfinite(o[0])) and np.all(np.isfinite(o[2]))


@pytest.mark.parametrize("geom,window,kv_dtype", [
    ((16, 8, 256), 0, F32),      # two query groups of 4 (8 rows per kv head each)
    ((16, 8, 256), 1024, F32),   # sliding window
    ((16, 2, 512), 0, BF16),     # 8 q heads per kv head: one query per group
], ids=["s256-f32", "s256-window", "g512-bf16"])
def test_verify_per_sequence_query_counts(gpu, geom, window, kv_dtype):
    # pkv_verify: every sequence its own draft length (the engine's verify_b = drafts + 1,
    # fewer after an early stop), including none. Rows past a sequence's count keep what
    # the caller left there; an invalid count gives NaN rows.
    print(f"[verify] per-sequence q_len {geom} window={window} {kv_dtype}", flush=True)
    hq, hkv, d = geom
    rng = np.random.default_rng(hq + hkv + d + window)
    bs, B, qmax = 16, 8, 5
    q_lens = np.array([1, 5, 3, 0, 4, 2, 5, 7], np.int32)  # the last one is invalid (> 5)
    ctx = rng.integers(300, 2500, B)
    kvs = hkv * d
    blocks_per = [(int(c) + qmax + bs - 1) // bs for c in ctx]
    nb = sum(blocks_per) + 8
    stride = max(blocks_per) + 2
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride), np.int32)
    lens = np.zeros(B, np.int32)
    off = 0
    for s in range(B):
        tables[s, :blocks_per[s]] = perm[off:off + blocks_per[s]]
        lens[s] = blocks_per[s]
        off += blocks_per[s]
    k = rng.standard_normal(nb * bs * kvs, dtype=np.float32)
    v = rng.standard_normal(nb * bs * kvs, dtype=np.float32)
    if kv_dtype == BF16:
        k, v = O.to_bf16(k), O.to_bf16(v)
    q = rng.standard_normal((B, qmax, hq, d), dtype=np.float32)
    pos = np.asarray(ctx, np.int32)
    p = make_params(LayerSpec(hq, hkv, d, window, kv_dtype), bs, nb, 0.0625)
    import ctypes
    max_pos = int(pos.max()) + qmax - 1
    ws_bytes = lib.load().pkv_workspace_size(ctypes.byref(p), B, qmax, max_pos)
    ws = hip.DeviceArray((ws_bytes,), np.uint8, zero=True)
    dk, dv = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    dt, dq = hip.DeviceArray.from_numpy(tables), hip.DeviceArray.from_numpy(q)
    dpos, dql = hip.DeviceArray.from_numpy(pos), hip.DeviceArray.from_numpy(q_lens)
    sentinel = np.full((B, qmax, hq, d), 12345.0, np.float32)
    out = hip.DeviceArray.from_numpy(sentinel)
    lib.call("pkv_verify", None, ctypes.byref(p), dq.ptr, dk.ptr, dv.ptr, dt.ptr, stride,
             dpos.ptr, dql.ptr, qmax, B, max_pos, out.ptr, ws.ptr, ws.nbytes)
    got = out.numpy()
    for s in range(B - 1):
        ql = int(q_lens[s])
        assert np.all(got[s, ql:] == 12345.0), f"sequence {s}: rows past its count written"
        if ql == 0:
            continue
        args = (q[s:s + 1, :ql], k, v, tables[s:s + 1], lens[s:s + 1], pos[s:s + 1], ql, hq,
                hkv, d, bs, window)
        ref = O.attend(*args, scale=0.0625)
        exact = None if kv_dtype == BF16 else O.attend_f64(
            q[s:s + 1, :ql], k, v, tables[s:s + 1], pos[s:s + 1], ql, hq, hkv, d, bs, window,
            scale=0.0625)
        parity.check(got[s:s + 1, :ql], ref, exact, bf16=kv_dtype == BF16, what=f"sequence {s}")
    assert np.all(np.isnan(got[B - 1])), "an invalid count gives NaN rows"
