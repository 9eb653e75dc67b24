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
    ((16, 8, 256), F32, 1),     # decode: fused
    ((16, 8, 256), BF16, 2),    # bf16, 4 rows: fused
    ((16, 2, 512), F32, 1),     # 8 rows per kv head at 512: fused (4 waves per head)
    ((16, 8, 256), F32, 4),     # fp64 MFMA verify: appends first
], ids=["f32-decode", "bf16-q2", "d512-g8", "mfma-verify"])
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
        # A sequence that ran out of blocks attends positions its append did not write,
        # through stale table entries (pkv.h: the one case where the fused launch may
        # read another sequence's row before or after its write); every other row matches.
        keep = st_s != lib.PKV_SEQ_OUT_OF_BLOCKS
        _same(out_f.numpy()[keep], out_s.numpy()[keep], f"{what}: outputs")
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
