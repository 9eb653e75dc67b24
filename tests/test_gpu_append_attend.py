"""pkv_append_attend against pkv_append followed by pkv_attend, on the device, step by step:
status, block tables, table lengths, free lists, every pool byte and the attention outputs
bit-identical. The batch mixes a sequence that opens a new block, one filling a partly
filled block, an inactive slot, a table entry outside the pool at the new token's block
(BAD_BLOCK) and a free list that runs short (OUT_OF_BLOCKS; such a sequence's output is
not compared, see pkv.h). Geometries cover the fused
launch (vector stream kernel: fp32 and bf16 at head_dim 256, fp32 at 512 with 8 rows per
kv head) and the path that appends first (the fp64 MFMA verify kernel)."""
import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, PagedKVCache, hip, lib

pytestmark = pytest.mark.gpu

BS = 16


def _caches(spec, B, nb, stride, q_len, tables, lens, free):
    out = []
    for _ in range(2):
        c = PagedKVCache([spec], block_size=BS, num_blocks=nb, max_seqs=B,
                         max_blocks_per_seq=stride, max_q_len=q_len, max_pos=stride * BS - 1,
                         scale=0.0625)
        c.tables.upload(tables)
        c.table_lens.upload(lens)
        fl = np.zeros(nb, np.int32)
        fl[:free.size] = free
        c.free_list.upload(fl)
        c.free_count.upload(np.array([free.size], np.int32))
        out.append(c)
    return out


def _values(rng, n, kv_dtype):
    """N(0,1) values in the pool dtype (bf16 as its bit patterns)."""
    x = rng.standard_normal(n, dtype=np.float32)
    if kv_dtype == BF16:
        return (x.view(np.uint32) >> 16).astype(np.uint16)  # truncated: finite bf16
    return x


def _same(a, b, what):
    assert np.array_equal(a, b, equal_nan=True), what


@pytest.mark.parametrize("geom,kv_dtype,q_len", [
    ((16, 8, 256), F32, 1),     # decode: fused, vector kernel
    ((16, 8, 256), BF16, 2),    # bf16, 4 rows: fused, vector kernel
    ((16, 2, 512), F32, 1),     # 8 rows per kv head at 512: fused, fp64 MFMA kernel
    ((16, 8, 256), F32, 4),     # verify, 8 rows per kv head: fused, fp64 MFMA kernel
    ((16, 2, 512), BF16, 1),    # bf16 at 512, 8 rows: fused, vector kernel (4 waves per head)
], ids=["f32-decode", "bf16-q2", "d512-g8", "mfma-verify", "d512-g8-bf16"])
def test_append_attend_matches_append_then_attend(gpu, geom, kv_dtype, q_len):
    print(f"[append_attend] {geom} {kv_dtype} q_len={q_len}", flush=True)
    rng = np.random.default_rng(q_len * 13 + geom[2])
    hq, hkv, d = geom
    B, stride = 6, 12
    spec = LayerSpec(hq, hkv, d, window=0, kv_dtype=kv_dtype)
    kvs = hkv * d
    # positions: a block boundary, mid-block, inactive, the bad-entry sequence, two more
    pos0 = np.array([32, 37, -1, 50, 95, 15], np.int32)
    lens = np.array([(max(p, 0) + BS - 1) // BS for p in pos0], np.int32)
    nb = int(lens.sum()) + 2  # two free blocks: later steps run short
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride), np.int32)
    o = 0
    for s in range(B):
        tables[s, :lens[s]] = perm[o:o + lens[s]]
        o += lens[s]
    free = np.sort(perm[o:])
    tables[3, 50 // BS] = nb + 7  # the block of sequence 3's next token: outside the pool
    fused, sep = _caches(spec, B, nb, stride, q_len, tables, lens, free)
    nelem = fused.k_pools[0].nbytes // (2 if kv_dtype == BF16 else 4)
    kp, vp = _values(rng, nelem, kv_dtype), _values(rng, nelem, kv_dtype)
    for c in (fused, sep):
        c.k_pools[0].upload(kp.reshape(c.k_pools[0].shape))
        c.v_pools[0].upload(vp.reshape(c.v_pools[0].shape))
    pos = pos0.copy()
    tok_off = (np.arange(B + 1) * q_len).astype(np.int32)
    for step in range(3):
        rows = B * q_len
        k_new = _values(rng, rows * kvs, kv_dtype).reshape(rows, kvs)
        v_new = _values(rng, rows * kvs, kv_dtype).reshape(rows, kvs)
        q = rng.standard_normal((B, q_len, hq, d), dtype=np.float32)
        dk, dv, dq = (hip.DeviceArray.from_numpy(x) for x in (k_new, v_new, q))
        out_f = hip.DeviceArray((B, q_len, hq, d), np.float32)
        out_s = hip.DeviceArray((B, q_len, hq, d), np.float32)
        st_f = fused.append_attend(0, pos, tok_off, dk, dv, q_len, rows, dq, q_len, out_f).numpy()
        st_s = sep.append(0, pos, tok_off, dk, dv, q_len, rows).numpy()
        sep.attend(0, dq, pos, q_len, out_s)
        what = f"step {step}"
        _same(st_f, st_s, f"{what}: status")
        a, b = fused.snapshot(), sep.snapshot()
        _same(a["tables"], b["tables"], f"{what}: tables")
        _same(a["table_lens"], b["table_lens"], f"{what}: table lengths")
        _same(a["free_list"], b["free_list"], f"{what}: free list")
        _same(fused.k_pools[0].numpy(), sep.k_pools[0].numpy(), f"{what}: K pool")
        _same(fused.v_pools[0].numpy(), sep.v_pools[0].numpy(), f"{what}: V pool")
        # A sequence that ran out of blocks is not attended by the fused call: NaN rows
        # (the separate calls attend positions its append did not write, through stale
        # table entries); every other row matches.
        keep = st_s != lib.PKV_SEQ_OUT_OF_BLOCKS
        got = out_f.numpy()
        _same(got[keep], out_s.numpy()[keep], f"{what}: outputs")
        assert np.all(np.isnan(got[~keep])), f"{what}: rows of a failed append"
        assert st_f[3] == lib.PKV_SEQ_BAD_BLOCK, "the out-of-pool entry is reported"
        pos = np.where(pos >= 0, pos + q_len, pos).astype(np.int32)
    fused.free()
    sep.free()


def test_append_attend_unsupported_geometry_changes_nothing(gpu):
    """A geometry the attention has no kernel for (32 q heads over 2 kv heads with 2
    queries: 32 rows per kv head) is refused before the append launches: tables, table
    lengths, the free list and every pool byte are unchanged."""
    print("[append_attend] unsupported geometry 32q/2kv q_len 2", flush=True)
    rng = np.random.default_rng(5)
    spec = LayerSpec(32, 2, 256, window=0)
    B, nb, stride, q_len = 3, 16, 8, 2
    c = PagedKVCache([spec], block_size=BS, num_blocks=nb, max_seqs=B, max_blocks_per_seq=stride,
                     max_q_len=q_len, max_pos=stride * BS - 1, scale=0.0625)
    kp = rng.standard_normal(c.k_pools[0].shape, dtype=np.float32)
    vp = rng.standard_normal(c.v_pools[0].shape, dtype=np.float32)
    c.k_pools[0].upload(kp)
    c.v_pools[0].upload(vp)
    before = c.snapshot()
    pos = np.array([16, 5, 31], np.int32)  # 16 and 31 + 1 open new blocks
    tok_off = (np.arange(B + 1) * q_len).astype(np.int32)
    rows = B * q_len
    dk = hip.DeviceArray.from_numpy(rng.standard_normal((rows, spec.kv_stride), dtype=np.float32))
    dv = hip.DeviceArray.from_numpy(rng.standard_normal((rows, spec.kv_stride), dtype=np.float32))
    dq = hip.DeviceArray.from_numpy(rng.standard_normal((B, q_len, 32, 256), dtype=np.float32))
    out = hip.DeviceArray((B, q_len, 32, 256), np.float32)
    with pytest.raises(lib.PkvError) as ei:
        c.append_attend(0, pos, tok_off, dk, dv, q_len, rows, dq, q_len, out)
    assert ei.value.code == lib.PKV_ERR_UNSUPPORTED
    after = c.snapshot()
    for key in ("tables", "table_lens", "free_list", "free_count"):
        _same(np.asarray(after[key]), np.asarray(before[key]), key)
    _same(c.k_pools[0].numpy(), kp, "K pool")
    _same(c.v_pools[0].numpy(), vp, "V pool")
    c.free()


@pytest.mark.parametrize("kv_dtype,q_len,geom", [
    (F32, 1, (16, 8, 256)),   # vector kernel
    (BF16, 2, (16, 8, 256)),  # vector kernel, two waves per kv head
    (F32, 4, (16, 8, 256)),   # fp64 MFMA kernel (8 rows per kv head)
    (F32, 1, (16, 2, 512)),   # fp64 MFMA kernel at the engine's global geometry
], ids=["f32-decode", "bf16-q2", "f32-q4-mfma", "g512-decode-mfma"])
def test_append_attend_allocation_follows_oracle(gpu, kv_dtype, q_len, geom):
    """The fused launch computes the block allocation itself (the merge launch writes the
    state): every status the allocation gives -- a new table, a block opened mid-batch,
    TABLE_FULL, an inactive slot, a free list that runs dry part-way (OUT_OF_BLOCKS),
    BAD_ARGS -- with status, tables, lengths, free list and count bit-exact against the
    oracle's block manager (O.CacheState) and the pools against its append; then a free
    count outside [0, num_blocks] (BAD_BLOCK for the sequences that need blocks, count
    left as is) against pkv_append + pkv_attend on a second cache. Outputs equal the two
    separate calls wherever the allocation gave OK; a sequence whose append failed is not
    attended and its rows are NaN (the engine skips its attention,
    model_speculative_moe_batched.mojo:1989-1992)."""
    print(f"[append_attend] allocation statuses {kv_dtype} q_len={q_len} geom={geom}", flush=True)
    rng = np.random.default_rng(40 + q_len)
    hq, hkv, d = geom
    B, stride, nb = 6, 3, 16
    spec = LayerSpec(hq, hkv, d, window=0, kv_dtype=kv_dtype)
    kvs = spec.kv_stride
    npdt = np.uint16 if kv_dtype == BF16 else np.float32
    lens = np.array([0, 1, 3, 0, 2, 1], np.int32)
    tables = np.zeros((B, stride), np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    o = 0
    for s in range(B):
        tables[s, :lens[s]] = perm[o:o + lens[s]]
        o += lens[s]
    # one block short of what the batch needs: the last sequence that needs one runs dry
    free = np.sort(perm[o:o + 2])
    # s0 new table; s1 opens block 1 (q_len 2) or stays in block 0; s2 TABLE_FULL;
    # s3 inactive; s4 opens block 2 (runs dry for q_len 2); s5 BAD_ARGS (rows past the end)
    pos = np.array([0, 16 - q_len + 1, stride * BS, -1, 32, 5], np.int32)
    if q_len == 1:
        pos[1] = 16  # opens block 1 too, so s4 runs dry in both variants
    rows = B * q_len
    tok_off = (np.arange(B + 1) * q_len).astype(np.int32)
    tok_off[B] = rows + 3  # s5's rows reach past total_rows
    kp = _values(rng, nb * BS * kvs, kv_dtype)
    vp = _values(rng, nb * BS * kvs, kv_dtype)

    def cache():
        c = PagedKVCache([spec], block_size=BS, num_blocks=nb, max_seqs=B,
                         max_blocks_per_seq=stride, max_q_len=q_len,
                         max_pos=stride * BS + q_len, scale=0.0625)
        c.tables.upload(tables)
        c.table_lens.upload(lens)
        fl = np.zeros(nb, np.int32)
        fl[:free.size] = free
        c.free_list.upload(fl)
        c.free_count.upload(np.array([free.size], np.int32))
        c.k_pools[0].upload(kp.reshape(c.k_pools[0].shape))
        c.v_pools[0].upload(vp.reshape(c.v_pools[0].shape))
        return c

    st = O.CacheState(1, kvs, BS, nb, B, stride, alloc_pools=False, dtype=npdt)
    st.k_pools[0], st.v_pools[0] = kp.copy(), vp.copy()
    st.tables[:] = tables
    st.table_lens[:] = lens
    st.bm.free_list[:free.size] = free
    st.bm.count[0] = free.size
    fused, sep = cache(), cache()
    k_new = _values(rng, (rows + 3) * kvs, kv_dtype).reshape(rows + 3, kvs)
    v_new = _values(rng, (rows + 3) * kvs, kv_dtype).reshape(rows + 3, kvs)
    q = rng.standard_normal((B, q_len, hq, d), dtype=np.float32)
    dk, dv, dq = (hip.DeviceArray.from_numpy(x) for x in (k_new, v_new, q))
    for rnd in range(2):
        out_f = hip.DeviceArray((B, q_len, hq, d), np.float32)
        out_s = hip.DeviceArray((B, q_len, hq, d), np.float32)
        if rnd == 1:  # a free count outside [0, num_blocks]: devices only
            pos = np.array([48 - q_len, 20, -1, -1, -1, -1], np.int32)
            tok_off = (np.arange(B + 1) * q_len).astype(np.int32)
            for c in (fused, sep):
                c.free_count.upload(np.array([nb + 5], np.int32))
        total = rows + 3 if rnd == 0 else rows
        st_f = fused.append_attend(0, pos, tok_off, dk, dv, q_len, total, dq, q_len, out_f).numpy()
        st_s = sep.append(0, pos, tok_off, dk, dv, q_len, total).numpy()
        sep.attend(0, dq, pos, q_len, out_s)
        a, b = fused.snapshot(), sep.snapshot()
        _same(st_f, st_s, f"round {rnd}: status vs pkv_append")
        for key in ("tables", "table_lens", "free_list", "free_count"):
            _same(np.asarray(a[key]), np.asarray(b[key]), f"round {rnd}: {key} vs pkv_append")
        _same(fused.k_pools[0].numpy(), sep.k_pools[0].numpy(), f"round {rnd}: K pool")
        _same(fused.v_pools[0].numpy(), sep.v_pools[0].numpy(), f"round {rnd}: V pool")
        ok = st_f == lib.PKV_SEQ_OK
        got = out_f.numpy()
        _same(got[ok], out_s.numpy()[ok], f"round {rnd}: outputs of OK sequences")
        failed = ~ok & (pos >= 0)
        assert failed.any(), "the round has a failed append"
        assert np.all(np.isnan(got[failed])), f"round {rnd}: failed appends give NaN rows"
        if rnd == 0:
            ref = st.append(0, pos, tok_off, k_new, v_new, q_len)
            _same(st_f, ref, "status vs oracle")
            assert list(ref) == [lib.PKV_SEQ_OK, lib.PKV_SEQ_OK, lib.PKV_SEQ_TABLE_FULL,
                                 lib.PKV_SEQ_OK, lib.PKV_SEQ_OUT_OF_BLOCKS,
                                 lib.PKV_SEQ_BAD_ARGS], list(ref)
            _same(a["tables"], st.tables, "tables vs oracle")
            _same(a["table_lens"], st.table_lens, "table lengths vs oracle")
            _same(a["free_list"], st.free_list, "free list vs oracle")
            _same(fused.k_pools[0].numpy().reshape(-1), st.k_pools[0], "K pool vs oracle")
            _same(fused.v_pools[0].numpy().reshape(-1), st.v_pools[0], "V pool vs oracle")
        else:
            assert list(st_f[:2]) == [lib.PKV_SEQ_BAD_BLOCK, lib.PKV_SEQ_OK], list(st_f)
            assert a["free_count"] == nb + 5
    fused.free()
    sep.free()
