"""GPU parity of the BASELINE.json configurations at their full sizes, through libpkv's C
ABI, against the oracle's restatement of the reference CPU path on the same inputs:
block tables, table lengths, free lists and every pool byte bit-exact; attention
outputs within the parity rule of tests/parity.py (1e-4 fp32, 2e-2 bf16).

  config 1  one sequence, append at 512 into a new block, attend 513 keys (fp32)
  config 3  8 x 32768-key decode over bf16 pages (split across workgroups)
  config 5  32 iterations of MTP shared-KV reads, 4-token verify append + causal
            attention on two layers, and rollback of rejected drafts (fp32)

Float data comes from the device-side seeded generator (pkv.synth) and is downloaded
for the oracle; the oracle replays the same appends / rollbacks on its own state.
Config 2 (the benchmark schedule) runs whole in test_gpu_config2.py."""
import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, PagedKVCache, hip
from pkv.workloads import LongDecode, SingleStep, VerifySchedule
from tests import parity

pytestmark = pytest.mark.gpu


def _cache(w, layers, kv_dtype, q_len):
    specs = [LayerSpec(w.HQ, w.HKV, w.D, window=w.WINDOW, kv_dtype=kv_dtype)
             for _ in range(layers)]
    cache = PagedKVCache(specs, block_size=w.BS, num_blocks=w.num_blocks, max_seqs=w.B,
                         max_blocks_per_seq=w.table_stride, max_q_len=q_len,
                         max_pos=w.max_pos, scale=w.SCALE)
    tables = np.zeros((w.B, w.table_stride), np.int32)
    tables[:, :w.tables0.shape[1]] = w.tables0
    cache.tables.upload(tables)
    cache.table_lens.upload(w.lens0)
    fl = np.zeros(w.num_blocks, np.int32)
    fl[:w.free0.size] = w.free0
    cache.free_list.upload(fl)
    cache.free_count.upload(np.array([w.free0.size], np.int32))
    return cache


def _oracle_state(w, layers, dtype):
    st = O.CacheState(layers, w.kv_stride, w.BS, w.num_blocks, w.B, w.table_stride,
                      dtype=dtype, alloc_pools=False)
    st.tables[:, :w.tables0.shape[1]] = w.tables0
    st.table_lens[:] = w.lens0
    st.bm.free_list[:w.free0.size] = w.free0
    st.bm.count[0] = w.free0.size
    return st


def _compare_state(cache, st, what):
    snap = cache.snapshot()
    assert np.array_equal(snap["table_lens"], st.table_lens), f"{what}: table lengths differ"
    for s in range(st.tables.shape[0]):
        n = int(st.table_lens[s])
        assert np.array_equal(snap["tables"][s, :n], st.tables[s, :n]), \
            f"{what}: block table of sequence {s} differs"
    assert np.array_equal(snap["free_list"], st.free_list), f"{what}: free lists differ"


def test_config1_single_step(gpu):
    print("[configs] config 1", flush=True)
    w = SingleStep(seed=1)
    d = w.device_data()
    cache = _cache(w, 1, F32, 1)
    cache.k_pools[0].copy_from(d["k"])
    cache.v_pools[0].copy_from(d["v"])
    st = _oracle_state(w, 1, np.float32)
    st.k_pools[0] = d["k"].numpy().reshape(-1).copy()
    st.v_pools[0] = d["v"].numpy().reshape(-1).copy()
    k_new, v_new, q = d["k_new"].numpy(), d["v_new"].numpy(), d["q"].numpy()
    status = cache.append(0, w.pos, [0, 1], d["k_new"], d["v_new"], 1, 1).numpy()
    assert status[0] == 0
    st.append(0, w.pos, [0, 1], k_new, v_new, 1)
    assert st.table_lens[0] == 33 and st.tables[0, 32] == w.free0[-1]  # LIFO back
    out = hip.DeviceArray((1, 1, w.HQ, w.D), np.float32)
    cache.attend(0, d["q"], w.pos, 1, out)
    _compare_state(cache, st, "config 1")
    assert np.array_equal(cache.k_pools[0].numpy().reshape(-1), st.k_pools[0])
    assert np.array_equal(cache.v_pools[0].numpy().reshape(-1), st.v_pools[0])
    ref = O.attend(q, st.k_pools[0], st.v_pools[0], st.tables, st.table_lens, w.pos, 1, w.HQ,
                   w.HKV, w.D, w.BS, 0, scale=w.SCALE)
    exact = O.attend_f64(q, st.k_pools[0], st.v_pools[0], st.tables, w.pos, 1, w.HQ, w.HKV,
                         w.D, w.BS, 0, scale=w.SCALE)
    parity.check(out.numpy(), ref, exact, what="config 1")
    cache.free()


def test_config3_long_context_bf16(gpu):
    print("[configs] config 3: 8 x 32768 keys, bf16 pages", flush=True)
    w = LongDecode(seed=3)
    d = w.device_data()
    cache = _cache(w, 1, BF16, 1)
    cache.k_pools[0].copy_from(d["k"])
    cache.v_pools[0].copy_from(d["v"])
    tok_off = np.arange(w.B + 1, dtype=np.int32)
    status = cache.append(0, w.pos, tok_off, d["k_new"], d["v_new"], 1, w.B).numpy()
    assert np.all(status == 0)
    out = hip.DeviceArray((w.B, 1, w.HQ, w.D), np.float32)
    cache.attend(0, d["q"], w.pos, 1, out)
    got = out.numpy()
    print("[configs] config 3: GPU done, running the oracle", flush=True)
    st = _oracle_state(w, 1, np.uint16)
    st.k_pools[0] = d["k"].numpy().reshape(-1)
    st.v_pools[0] = d["v"].numpy().reshape(-1)
    st.append(0, w.pos, tok_off, d["k_new"].numpy(), d["v_new"].numpy(), 1)
    _compare_state(cache, st, "config 3")
    assert np.array_equal(cache.k_pools[0].numpy().reshape(-1), st.k_pools[0]), "K pool"
    assert np.array_equal(cache.v_pools[0].numpy().reshape(-1), st.v_pools[0]), "V pool"
    ref = O.attend(d["q"].numpy(), st.k_pools[0], st.v_pools[0], st.tables, st.table_lens,
                   w.pos, 1, w.HQ, w.HKV, w.D, w.BS, 0, scale=w.SCALE,
                   nthreads=O.max_threads(), par=1)
    err, _ = parity.check(got, ref, bf16=True, what="config 3")
    print(f"[configs] config 3: max rel err {err:.3g}", flush=True)
    cache.free()


def test_config5_verify_rollback_shared_kv(gpu):
    print("[configs] config 5: 32 iterations of MTP read + verify + rollback", flush=True)
    w = VerifySchedule(seed=5)
    d = w.device_data()
    L, B, DR = w.LAYERS, w.B, w.DRAFT
    cache = _cache(w, L, F32, DR)
    st = _oracle_state(w, L, np.float32)
    for layer in range(L):
        for kv in range(2):
            pool = (cache.k_pools, cache.v_pools)[kv][layer]
            pool.copy_from(d["pools"][layer][kv])
            (st.k_pools, st.v_pools)[kv][layer] = d["pools"][layer][kv].numpy().reshape(-1).copy()
    q_all, mtp_all = d["q"].numpy(), d["mtp_q"].numpy()
    kn_all, vn_all = d["k_new"].numpy(), d["v_new"].numpy()
    qstep = B * DR * w.HQ * w.D * 4
    mstep = B * w.HQ * w.D * 4
    kvstep = B * DR * w.kv_stride * 4
    out_v = hip.DeviceArray((B, DR, w.HQ, w.D), np.float32)
    out_m = hip.DeviceArray((B, 1, w.HQ, w.D), np.float32)
    tok_off = w.tok_off()
    worst = 0.0
    for it in range(w.ITERS):
        pos = w.pos(it)
        # 1. MTP drafting reads the target pools at kv_pos = L - 1 (read only); the first
        #    and last draft step of every fourth iteration are checked against the oracle.
        for dstep in range(DR):
            for layer in range(L):
                n = it * L + layer
                cache.attend(layer, d["mtp_q"].ptr + (n * DR + dstep) * mstep, pos - 1, 1,
                             out_m)
                if it % 4 == 0 and dstep in (0, DR - 1):
                    qm = mtp_all[n, dstep]
                    ref = O.attend(qm, st.k_pools[layer], st.v_pools[layer], st.tables,
                                   st.table_lens, pos - 1, 1, w.HQ, w.HKV, w.D, w.BS, 0,
                                   scale=w.SCALE, nthreads=O.max_threads(), par=1)
                    ex = O.attend_f64(qm, st.k_pools[layer], st.v_pools[layer], st.tables,
                                      pos - 1, 1, w.HQ, w.HKV, w.D, w.BS, 0, scale=w.SCALE)
                    parity.check(out_m.numpy(), ref, ex, what=f"it {it} mtp {dstep} layer {layer}")
        # 2. verify: append the draft rows on both layers, attend 4 causal queries
        for layer in range(L):
            n = it * L + layer
            status = cache.append(layer, pos, tok_off, d["k_new"].ptr + n * kvstep,
                                  d["v_new"].ptr + n * kvstep, DR, B * DR).numpy()
            assert np.all(status == 0), f"it {it}: append status {status}"
            st.append(layer, pos, tok_off, kn_all[n], vn_all[n], DR)
        _compare_state(cache, st, f"it {it} after append")
        for layer in range(L):
            n = it * L + layer
            cache.attend(layer, d["q"].ptr + n * qstep, pos, DR, out_v)
            ref = O.attend(q_all[n], st.k_pools[layer], st.v_pools[layer], st.tables,
                           st.table_lens, pos, DR, w.HQ, w.HKV, w.D, w.BS, 0, scale=w.SCALE,
                           nthreads=O.max_threads(), par=1)
            ex = O.attend_f64(q_all[n], st.k_pools[layer], st.v_pools[layer], st.tables, pos,
                              DR, w.HQ, w.HKV, w.D, w.BS, 0, scale=w.SCALE)
            e32, _ = parity.check(out_v.numpy(), ref, ex, what=f"it {it} verify layer {layer}")
            worst = max(worst, e32)
        # 3. acceptance -> rollback of the rejected drafts
        new_len = w.new_len(it)
        status = cache.rollback(new_len).numpy()
        assert np.all(status == 0), f"it {it}: rollback status {status}"
        st.rollback(new_len)
        _compare_state(cache, st, f"it {it} after rollback")
        assert np.array_equal(st.table_lens, (new_len + w.BS - 1) // w.BS)
        if it % 8 == 7:
            print(f"[configs] config 5: iteration {it + 1} ok, worst err {worst:.3g}", flush=True)
    for layer in range(L):
        assert np.array_equal(cache.k_pools[layer].numpy().reshape(-1), st.k_pools[layer])
        assert np.array_equal(cache.v_pools[layer].numpy().reshape(-1), st.v_pools[layer])
    cache.free()
