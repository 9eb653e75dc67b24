"""GPU parity of K3 (chunked-prefill MFMA attention, bf16 pages) against the oracle's
restatement of the engine's per-token prefill: append the chunk's K/V, then one
paged_attention_layer call per chunk token (…batched.mojo:2600-2637, :2767-2833), run
on the same bf16-rounded values (Q upcast exactly to fp32). Outputs within 2e-2
(max |x - ref| / (|ref| + 1e-3)); cache state after the append bit-exact."""
import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, LayerSpec, PagedKVCache, hip
from pkv.workloads import PrefillChunk
from tests import parity

pytestmark = pytest.mark.gpu


def _run(w, seed_rows=None, check_state=True, q_counts=None):
    """Appends each sequence's chunk (q_counts[s] tokens, default CHUNK) at its prefix
    end, runs pkv_prefill, and checks state and outputs against the oracle."""
    B = w.B
    counts = np.full(B, w.CHUNK, np.int64) if q_counts is None else np.asarray(q_counts)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    rows = int(off[-1])
    spec = LayerSpec(w.HQ, w.HKV, w.D, window=w.WINDOW, kv_dtype=BF16)
    cache = PagedKVCache([spec], block_size=w.BS, num_blocks=w.num_blocks, max_seqs=B,
                         max_blocks_per_seq=w.table_stride, max_pos=w.max_pos, scale=w.SCALE)
    d = w.device_data()
    cache.k_pools[0].copy_from(d["k"])
    cache.v_pools[0].copy_from(d["v"])
    tables = np.zeros((B, w.table_stride), np.int32)
    tables[:, :w.tables0.shape[1]] = w.tables0
    cache.tables.upload(tables)
    cache.table_lens.upload(w.lens0)
    fl = np.zeros(w.num_blocks, np.int32)
    fl[:w.free0.size] = w.free0
    cache.free_list.upload(fl)
    cache.free_count.upload(np.array([w.free0.size], np.int32))
    st = O.CacheState(1, w.kv_stride, w.BS, w.num_blocks, B, w.table_stride, dtype=np.uint16,
                      alloc_pools=False)
    st.k_pools[0] = d["k"].numpy().reshape(-1)
    st.v_pools[0] = d["v"].numpy().reshape(-1)
    st.tables[:] = tables
    st.table_lens[:] = w.lens0
    st.bm.free_list[:w.free0.size] = w.free0
    st.bm.count[0] = w.free0.size
    kn = d["k_new"].numpy().reshape(-1, w.kv_stride)[:max(rows, 1)]
    vn = d["v_new"].numpy().reshape(-1, w.kv_stride)[:max(rows, 1)]
    max_q = int(counts.max())
    status = cache.append(0, w.pos, off, d["k_new"], d["v_new"], max_q, rows).numpy()
    assert np.all(status == 0), status
    st.append(0, w.pos, off, kn, vn, max_q)
    out = hip.DeviceArray((max(rows, 1), w.HQ, w.D), np.float32)
    cache.prefill(0, d["q"], w.pos, off, max_q, out)
    got = out.numpy()
    if check_state:
        snap = cache.snapshot()
        assert np.array_equal(snap["tables"], st.tables)
        assert np.array_equal(snap["table_lens"], st.table_lens)
        assert np.array_equal(snap["free_list"], st.free_list)
        assert np.array_equal(cache.k_pools[0].numpy().reshape(-1), st.k_pools[0])
        assert np.array_equal(cache.v_pools[0].numpy().reshape(-1), st.v_pools[0])
    q32 = O.bf16_to_f32(d["q"].numpy().reshape(-1, w.HQ, w.D)[:max(rows, 1)])
    worst = 0.0
    for s in range(B):
        n = int(counts[s])
        if n == 0:
            continue
        qs = q32[off[s]:off[s + 1]].reshape(1, n, w.HQ, w.D)
        ref = O.attend(qs, st.k_pools[0], st.v_pools[0], st.tables[s:s + 1],
                       st.table_lens[s:s + 1], w.pos[s:s + 1], n, w.HQ, w.HKV, w.D, w.BS,
                       w.WINDOW, scale=w.SCALE, nthreads=O.max_threads(), par=2)
        e, _ = parity.check(got[off[s]:off[s + 1]], ref.reshape(n, w.HQ, w.D), bf16=True,
                            what=f"sequence {s} (prefix {w.pos[s]}, {n} queries)")
        worst = max(worst, e)
    cache.free()
    return worst


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4)], ids=["G2", "G1", "G4"])
@pytest.mark.parametrize("window", [0, 100])
def test_prefill_small_ragged(gpu, hq, hkv, window):
    print(f"[prefill] small hq={hq} hkv={hkv} window={window}", flush=True)
    w = PrefillChunk(seed=hq + hkv + window, batch=5, chunk=200, prefix_max=300, hq=hq,
                     hkv=hkv, window=window, prefix=[0, 5, 16, 100, 300])
    # ragged chunk lengths: one query, a partial 64-key tile, exact tiles, a long one
    _run(w, q_counts=[1, 17, 64, 130, 200])


@pytest.mark.parametrize("bs", [8, 32, 64])
def test_prefill_block_sizes(gpu, bs):
    """Each wave copies eight keys of a tile from one block: block sizes 8 (exactly one
    block), 32 and 64 (a wave's keys start inside a block)."""
    print(f"[prefill] block_size {bs}", flush=True)

    class Chunk(PrefillChunk):
        BS = bs

    w = Chunk(seed=bs, batch=4, chunk=160, prefix_max=400, prefix=[0, 9, 77, 400])
    _run(w, q_counts=[3, 64, 100, 160])


def test_prefill_config4_full(gpu):
    print("[prefill] config 4: 4 x 2048-token chunks over prefixes up to 6144", flush=True)
    w = PrefillChunk(seed=4)
    worst = _run(w)
    print(f"[prefill] config 4 worst rel err {worst:.3g}", flush=True)


def test_prefill_inactive_bad_table_and_overflow(gpu):
    print("[prefill] inactive / bad table / max_q overflow", flush=True)
    import ctypes

    from pkv import lib
    from pkv.engine import make_params

    rng = np.random.default_rng(9)
    hq, hkv, d, bs, nb = 16, 8, 256, 16, 64
    spec = LayerSpec(hq, hkv, d, kv_dtype=BF16)
    p = make_params(spec, bs, nb, 0.0625)
    stride = 16
    tables = rng.integers(0, nb, (3, stride)).astype(np.int32)
    tables[2, 0] = nb + 3  # outside the pool (sequence 2 reads block 0 only)
    kp = hip.DeviceArray((nb * bs * hkv * d,), np.uint16, zero=True)
    q = hip.DeviceArray.from_numpy(O.to_bf16(rng.standard_normal((30, hq, d), dtype=np.float32)))
    pos = np.array([10, -1, 5], np.int32)
    q_off = np.array([0, 10, 20, 30], np.int32)
    out = hip.DeviceArray((30, hq, d), np.float32)
    dt, dp, do = (hip.DeviceArray.from_numpy(x) for x in (tables, pos, q_off))
    lib.call("pkv_prefill", None, ctypes.byref(p), q.ptr, kp.ptr, kp.ptr, dt.ptr, stride, dp.ptr,
             do.ptr, 10, 3, 200, out.ptr)
    o = out.numpy()
    assert np.all(o[:10] == 0.0)  # zero V rows
    assert np.all(o[10:20] == 0.0)  # inactive sequence
    assert np.all(np.isnan(o[20:30]))  # bad table entry
    # a sequence with more queries than max_q: NaN for all of its rows
    q_off2 = np.array([0, 10, 10, 30], np.int32)
    pos2 = np.array([10, -1, 5], np.int32)
    tables2 = np.clip(tables, 0, nb - 1)
    dt2, dp2, do2 = (hip.DeviceArray.from_numpy(x) for x in (tables2, pos2, q_off2))
    lib.call("pkv_prefill", None, ctypes.byref(p), q.ptr, kp.ptr, kp.ptr, dt2.ptr, stride,
             dp2.ptr, do2.ptr, 10, 3, 200, out.ptr)
    o = out.numpy()
    assert np.all(np.isfinite(o[:10])) and np.all(np.isnan(o[10:30]))
