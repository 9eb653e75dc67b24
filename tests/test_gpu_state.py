"""GPU parity of K1 (fused allocate + scatter) and K5 (rollback / retire) against the
oracle's restatement of the engine's bookkeeping: block tables, table lengths, the free
list and every pool byte must match bit-exactly."""
import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, PagedKVCache, hip, lib

pytestmark = pytest.mark.gpu


def _compare(cache: PagedKVCache, st: O.CacheState, layers=(0,), pools=True):
    snap = cache.snapshot()
    np.testing.assert_array_equal(snap["table_lens"], st.table_lens)
    np.testing.assert_array_equal(snap["tables"], st.tables)
    np.testing.assert_array_equal(snap["free_list"], st.free_list)
    if pools:
        for l in layers:
            np.testing.assert_array_equal(cache.k_pools[l].numpy().reshape(-1), st.k_pools[l])
            np.testing.assert_array_equal(cache.v_pools[l].numpy().reshape(-1), st.v_pools[l])


def _mk(kv_dtype, nseq, bs, num_blocks, stride, kvh=2, d=64, layers=1):
    spec = LayerSpec(num_heads=kvh * 2, num_kv_heads=kvh, head_dim=d, kv_dtype=kv_dtype)
    cache = PagedKVCache([spec] * layers, block_size=bs, num_blocks=num_blocks, max_seqs=nseq,
                         max_blocks_per_seq=stride)
    st = O.CacheState(layers, spec.kv_stride, bs, num_blocks, nseq, stride,
                      dtype=np.uint16 if kv_dtype == BF16 else np.float32)
    return spec, cache, st


@pytest.mark.parametrize("kv_dtype", [F32, BF16])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_append_rollback_sequences(gpu, kv_dtype, seed):
    print(f"[state] kv={kv_dtype} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    nseq, bs, num_blocks, stride, max_new = 7, 4, 40, 24, 9
    spec, cache, st = _mk(kv_dtype, nseq, bs, num_blocks, stride, layers=2)
    length = np.zeros(nseq, np.int64)
    npdt = np.uint16 if kv_dtype == BF16 else np.float32
    kd = hip.DeviceArray((nseq * max_new, spec.kv_stride), npdt)
    vd = hip.DeviceArray((nseq * max_new, spec.kv_stride), npdt)
    for step in range(40):
        if rng.random() < 0.7:
            n_new = rng.integers(0, max_new + 1, nseq).astype(np.int32)
            pos = length.astype(np.int32).copy()
            pos[rng.random(nseq) < 0.1] = -1  # inactive slots
            off = O.ragged_tok_off(n_new)
            rows = max(int(off[-1]), 1)
            raw = rng.standard_normal((2, rows, spec.kv_stride)).astype(np.float32)
            k = O.to_bf16(raw[0]) if kv_dtype == BF16 else raw[0]
            v = O.to_bf16(raw[1]) if kv_dtype == BF16 else raw[1]
            kd.upload_at(0, k)
            vd.upload_at(0, v)
            layer = int(rng.integers(0, 2))
            ref_status = st.append(layer, pos, off, k, v, max_new)
            status = cache.append(layer, pos, off, kd, vd, max_new, rows).numpy()
            np.testing.assert_array_equal(status, ref_status, err_msg=f"step {step}")
            ok = (ref_status == 0) & (pos >= 0)
            length[ok] += n_new[ok]
        else:
            new_len = np.full(nseq, -1, np.int32)
            pick = rng.random(nseq) < 0.5
            new_len[pick] = [rng.integers(0, length[s] + 1) for s in np.nonzero(pick)[0]]
            length[pick] = new_len[pick]
            st.rollback(new_len)
            cache.rollback(new_len)
        _compare(cache, st, layers=(0, 1), pools=(step % 5 == 4))
    _compare(cache, st, layers=(0, 1))
    cache.free()


def test_out_of_blocks_and_table_full(gpu):
    print("[state] oom / table full", flush=True)
    nseq, bs, num_blocks, stride = 4, 4, 6, 3
    spec, cache, st = _mk(F32, nseq, bs, num_blocks, stride)
    k = np.arange(nseq * 13 * spec.kv_stride, dtype=np.float32).reshape(nseq * 13, -1)
    kd, vd = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(-k)
    pos = np.array([0, 0, 0, 0], np.int32)
    n_new = np.array([5, 13, 9, 2], np.int32)  # needs 2, 4 (> stride 3: full), 3, 1
    off = O.ragged_tok_off(n_new)
    ref = st.append(0, pos, off, k, -k, 13)
    got = cache.append(0, pos, off, kd, vd, 13, nseq * 13).numpy()
    np.testing.assert_array_equal(got, ref)
    assert list(ref) == [lib.PKV_SEQ_OK, lib.PKV_SEQ_TABLE_FULL, lib.PKV_SEQ_OK, lib.PKV_SEQ_OK]
    _compare(cache, st)
    # The pool now has 0 free blocks: a second round runs dry part-way.
    pos2 = np.array([5, -1, 9, 2], np.int32)
    off2 = O.ragged_tok_off([4, 0, 4, 7])
    ref = st.append(0, pos2, off2, k, -k, 13)
    got = cache.append(0, pos2, off2, kd, vd, 13, nseq * 13).numpy()
    np.testing.assert_array_equal(got, ref)
    assert lib.PKV_SEQ_OUT_OF_BLOCKS in list(ref)
    _compare(cache, st)
    # Token ranges outside the new rows or longer than max_new are rejected unchanged.
    off3 = np.array([0, 2, 60, 60, 60], np.int32)
    ref = st.append(0, np.array([1, 0, 3, 3], np.int32), off3, k, -k, 13)
    got = cache.append(0, np.array([1, 0, 3, 3], np.int32), off3, kd, vd, 13, 52).numpy()
    np.testing.assert_array_equal(got, ref)
    assert ref[1] == lib.PKV_SEQ_BAD_ARGS
    _compare(cache, st)
    cache.free()


def test_config1_append_into_new_block(gpu):
    # Config 1 bookkeeping: 256-block pool, the sequence owns a seeded permutation prefix
    # of 32 blocks (512 tokens); appending at pos 512 pops the LIFO back of the free list.
    print("[state] config 1 append", flush=True)
    rng = np.random.default_rng(1)
    bs, nb = 16, 256
    spec = LayerSpec(16, 8, 256)
    cache = PagedKVCache([spec], block_size=bs, num_blocks=nb, max_seqs=1, max_blocks_per_seq=64)
    st = O.CacheState(1, spec.kv_stride, bs, nb, 1, 64)
    perm = rng.permutation(nb).astype(np.int32)
    table = perm[:32]
    free = np.sort(perm[32:]).astype(np.int32)
    st.tables[0, :32] = table
    st.table_lens[0] = 32
    st.bm.free_list[:free.size] = free
    st.bm.count[0] = free.size
    cache.tables.upload(st.tables)
    cache.table_lens.upload(st.table_lens)
    fl = np.zeros(nb, np.int32)
    fl[:free.size] = free
    cache.free_list.upload(fl)
    cache.free_count.upload(np.array([free.size], np.int32))
    k = rng.standard_normal((1, 1, spec.kv_stride)).astype(np.float32)
    v = rng.standard_normal((1, 1, spec.kv_stride)).astype(np.float32)
    st.append(0, [512], [0, 1], k, v, 1)
    dk, dv = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    cache.append(0, [512], [0, 1], dk, dv, 1, 1)
    assert st.table_lens[0] == 33 and st.tables[0, 32] == free[-1]
    _compare(cache, st)
    cache.free()


@pytest.mark.parametrize("entry", ["append", "append_attend"])
def test_bad_table_entry_skips_only_its_rows(gpu, entry):
    """A 40-token append (ten scatter workgroups of 4 tokens at 8 KiB rows) over three
    blocks, the middle one's table entry outside the pool: status BAD_BLOCK, the rows of
    that block are skipped and every other row is written, whichever workgroup copies it.
    The allocation and the other sequences follow the oracle bit-exactly. The oracle runs
    the same call with a spare in-pool block in place of the bad entry; the device pools
    must equal the oracle's everywhere except that spare block, which stays untouched.
    append_attend: the fused launch copies the rows and attends (outputs against pkv_append
    + pkv_attend)."""
    print(f"[state] bad table entry, {entry}", flush=True)
    rng = np.random.default_rng(11)
    bs, nb, stride, nseq = 16, 14, 6, 3
    spare = nb - 1  # in the pool, in no table and not on the free list
    spec = LayerSpec(16, 8, 256)
    kvs = spec.kv_stride
    tables = np.zeros((nseq, stride), np.int32)
    tables[0, :2] = [4, 9]
    tables[1, :1] = [2]
    tables[2, :2] = [7, 0]
    lens = np.array([2, 1, 2], np.int32)
    free = np.array([1, 3, 5, 6, 8, 10, 11, 12], np.int32)
    dev_tables = tables.copy()
    dev_tables[0, 1] = nb + 3  # outside the pool
    tables[0, 1] = spare
    pos = np.array([5, 3, 30], np.int32)
    n_new = np.array([40, 6, 5], np.int32)  # blocks 0-2 of seq 0, block 0 of 1, 1-2 of 2
    off = O.ragged_tok_off(n_new)
    rows = int(off[-1])
    k = rng.standard_normal((rows, kvs), dtype=np.float32)
    v = rng.standard_normal((rows, kvs), dtype=np.float32)
    kp = rng.standard_normal(nb * bs * kvs, dtype=np.float32)
    vp = rng.standard_normal(nb * bs * kvs, dtype=np.float32)

    def device_cache():
        c = PagedKVCache([spec], block_size=bs, num_blocks=nb, max_seqs=nseq,
                         max_blocks_per_seq=stride, max_pos=stride * bs - 1, scale=0.0625)
        c.tables.upload(dev_tables)
        c.table_lens.upload(lens)
        fl = np.zeros(nb, np.int32)
        fl[:free.size] = free
        c.free_list.upload(fl)
        c.free_count.upload(np.array([free.size], np.int32))
        c.k_pools[0].upload(kp.reshape(c.k_pools[0].shape))
        c.v_pools[0].upload(vp.reshape(c.v_pools[0].shape))
        return c

    st = O.CacheState(1, kvs, bs, nb, nseq, stride, alloc_pools=False)
    st.k_pools[0], st.v_pools[0] = kp.copy(), vp.copy()
    st.tables[:] = tables
    st.table_lens[:] = lens
    st.bm.free_list[:free.size] = free
    st.bm.count[0] = free.size
    ref = st.append(0, pos, off, k, v, int(n_new.max()))
    dk, dv = hip.DeviceArray.from_numpy(k), hip.DeviceArray.from_numpy(v)
    a = device_cache()
    got = a.append(0, pos, off, dk, dv, int(n_new.max()), rows).numpy()
    q = rng.standard_normal((nseq, 1, 16, 256), dtype=np.float32)
    dq = hip.DeviceArray.from_numpy(q)
    if entry == "append_attend":
        out_ref = hip.DeviceArray((nseq, 1, 16, 256), np.float32)
        a.attend(0, dq, pos, 1, out_ref)
        out = hip.DeviceArray((nseq, 1, 16, 256), np.float32)
        b = device_cache()
        got_b = b.append_attend(0, pos, off, dk, dv, int(n_new.max()), rows, dq, 1, out).numpy()
        np.testing.assert_array_equal(got_b, got)
        np.testing.assert_array_equal(out.numpy(), out_ref.numpy())  # block 0 only: no NaN
        a.free()
        a = b
    assert list(got) == [lib.PKV_SEQ_BAD_BLOCK, lib.PKV_SEQ_OK, lib.PKV_SEQ_OK]
    assert list(ref) == [0, 0, 0]
    snap = a.snapshot()
    exp_tables = st.tables.copy()
    exp_tables[0, 1] = nb + 3
    np.testing.assert_array_equal(snap["tables"], exp_tables)
    np.testing.assert_array_equal(snap["table_lens"], st.table_lens)
    np.testing.assert_array_equal(snap["free_list"], st.free_list)
    row_elems = bs * kvs
    for name, dev, exp, init in (("K", a.k_pools[0], st.k_pools[0], kp),
                                 ("V", a.v_pools[0], st.v_pools[0], vp)):
        g = dev.numpy().reshape(-1)
        sl = slice(spare * row_elems, (spare + 1) * row_elems)
        np.testing.assert_array_equal(g[sl], init[sl], err_msg=f"{name}: the bad block's rows")
        e = exp.copy()
        e[sl] = init[sl]
        np.testing.assert_array_equal(g, e, err_msg=f"{name} pool")
    a.free()
