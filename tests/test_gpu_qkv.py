"""GPU parity of the fused producer step + append (pkv_append_qkv) against the oracle's
restatement (pkvo_append_qkv: rms_norm / rms_norm_noscale per head, apply_rope_qk, then
the append; …batched.mojo:1974-2001, attention.mojo:69-132). Block tables, table
lengths, free lists and statuses are bit-exact, and pool rows the append does not address
are untouched (bit-exact). The normalised, rotated values follow tests/parity.py's rule
(max |x - ref| / (|ref| + 1e-3)): fp32 within 1e-4 of the fp32 oracle -- or within its own
distance from exact where that is larger -- and within 1e-5 of the float64 producer;
bf16 within 2e-2 of the oracle. (cos / sin and the last bit of the norms are not pinned
to the reference's bits.) The prefill case chains the producer into pkv_prefill."""
import numpy as np
import pytest

from oracle import oracle as O
from pkv import BF16, F32, LayerSpec, PagedKVCache, hip, lib
from tests import parity

pytestmark = pytest.mark.gpu


def _inputs(rng, n_new, hq, hkv, D, with_v):
    tok_off = O.ragged_tok_off(n_new)
    rows = max(int(tok_off[-1]), 1)
    q = (rng.standard_normal((rows, hq * D)) * 2).astype(np.float32)
    k = (rng.standard_normal((rows, hkv * D)) * 2).astype(np.float32)
    v = rng.standard_normal((rows, hkv * D)).astype(np.float32) if with_v else None
    qw = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    kw = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    return tok_off, rows, q, k, v, qw, kw


def _dev(*arrs):
    return [None if a is None else hip.DeviceArray.from_numpy(a) for a in arrs]


def _close(got, want, bf16, what):
    if bf16:
        got, want = O.bf16_to_f32(got), O.bf16_to_f32(want)
    tol = parity.TOL_BF16 if bf16 else parity.TOL_F32
    err = O.max_rel_err(got, want)
    assert err <= tol, f"{what}: max rel err {err} > {tol}"
    return err


def _written_rows(st, pos, tok_off, status, slots):
    """(pool row, input row) of every K / V row the append wrote, from the oracle's state
    after its append: pages through the tables, rings through ring_row (the last
    ring_size tokens of a call)."""
    out = []
    for s in range(pos.size):
        n = int(tok_off[s + 1] - tok_off[s])
        if status[s] != 0 or pos[s] < 0 or n <= 0:
            continue
        for b in range(n):
            p = int(pos[s]) + b
            if isinstance(st, O.RingState):
                if b < n - st.ring_size:
                    continue
                row = O.ring_row(int(slots[s]), st.ring_size, p)
            else:
                row = int(st.tables[s, p // st.block_size]) * st.block_size + p % st.block_size
            out.append((row, int(tok_off[s]) + b))
    return out


def _check_values(got, ref, exact, bf16, what):
    if bf16:
        _close(got, ref, True, what)
    else:
        parity.check(got, ref, exact, what=what)


def _run(cache, st, layer, pos, n_new, hq, hkv, D, is_global, with_v, q_bf16, rng, slots=None,
         q_in_place=False):
    tok_off, rows, q, k, v, qw, kw = _inputs(rng, n_new, hq, hkv, D, with_v)
    dq, dk, dv, dqw, dkw = _dev(q, k, v, qw, kw)
    if q_in_place:
        q_out = dq
    else:
        q_out = hip.DeviceArray((rows, hq * D), np.uint16 if q_bf16 else np.float32, zero=True)
    max_new = int(max(n_new.max(), 1))
    before = [cache.k_pools[layer].numpy(), cache.v_pools[layer].numpy()]
    status = cache.append_qkv(layer, pos, tok_off, dq, dk, dv, dqw, dkw, q_out, max_new, rows,
                              is_global, BF16 if q_bf16 else F32, batch=pos.size).numpy()
    want_st, want_q = O.append_qkv(st, 0, pos, tok_off, q, k, v, qw, kw, max_new, hq, hkv, D,
                                   is_global, slots=slots)
    ex_q, ex_k, ex_v = O.producer_f64(pos, tok_off, q, k, v, qw, kw, max_new, hq, hkv, D,
                                      is_global)
    assert np.array_equal(status[:pos.size], want_st), (status, want_st)
    got_q = q_out.numpy()
    valid = np.isfinite(want_q)
    if q_bf16:
        _close(got_q[valid], O.to_bf16(want_q[valid]), True, "q_out")
    else:
        parity.check(got_q[valid], want_q[valid], ex_q[valid], what="q_out")
    # K / V pools: addressed rows within the rule, every other row untouched
    bf16 = st.dtype == np.uint16
    wr = _written_rows(st, pos, tok_off, want_st, slots)
    prow = np.array([w[0] for w in wr], np.int64)
    irow = np.array([w[1] for w in wr], np.int64)
    kvs = hkv * D
    for name, dev, host, ex, prev in (("K", cache.k_pools[layer], st.k_pools[0], ex_k, before[0]),
                                      ("V", cache.v_pools[layer], st.v_pools[0], ex_v, before[1])):
        cur = dev.numpy().reshape(-1, kvs)
        prev = prev.reshape(-1, kvs)
        keep = np.ones(cur.shape[0], bool)
        keep[prow] = False
        assert np.array_equal(cur[keep], prev[keep]), f"{name}: rows outside the append changed"
        if prow.size:
            _check_values(cur[prow], host.reshape(-1, kvs)[prow], ex[irow], bf16, f"{name} rows")
    return q_out, tok_off


def _state_match(cache, st):
    snap = cache.snapshot()
    assert np.array_equal(snap["table_lens"], st.table_lens)
    assert np.array_equal(snap["free_list"], st.free_list)
    for s in range(st.tables.shape[0]):
        n = int(st.table_lens[s])
        assert np.array_equal(snap["tables"][s, :n], st.tables[s, :n])


@pytest.mark.parametrize("is_global,hq,hkv,D,kv_dtype,with_v,q_bf16", [
    (False, 16, 8, 256, F32, True, False),   # sliding layer, fp32 pools
    (True, 16, 2, 512, BF16, False, True),   # global layer, V := K, bf16 pools and Q
    (True, 16, 8, 256, F32, True, False),    # the configs' 16/8/256 global stand-in
    (False, 6, 3, 256, BF16, True, True),    # odd kv heads: one head per wave, not pairs
], ids=["sliding-f32", "global512-bf16", "global256-f32", "odd-heads-256-bf16"])
def test_append_qkv_decode_and_chunks(gpu, is_global, hq, hkv, D, kv_dtype, with_v, q_bf16):
    print(f"[qkv] global={is_global} {hq}/{hkv}/{D} {kv_dtype}", flush=True)
    rng = np.random.default_rng(D + hkv)
    B, nb, stride, bs = 6, 64, 6300, 16
    spec = LayerSpec(hq, hkv, D, window=0 if is_global else 1024, kv_dtype=kv_dtype)
    cache = PagedKVCache([spec], block_size=bs, num_blocks=nb, max_seqs=B,
                         max_blocks_per_seq=stride, max_pos=stride * bs - 1)
    npdt = np.uint16 if kv_dtype == BF16 else np.float32
    st = O.CacheState(1, hkv * D, bs, nb, B, stride, dtype=npdt)
    # Sequence 5 sits at position 100000 (the reference's largest RoPE test position):
    # its table already holds 6250 entries (all block 0, never written here), so the
    # append takes one block.
    tables = np.zeros((B, stride), np.int32)
    lens = np.zeros(B, np.int32)
    lens[5] = 100000 // bs
    cache.tables.upload(tables)
    cache.table_lens.upload(lens)
    st.table_lens[:] = lens
    pos = np.array([0, 15, 16, 333, 4095, 100000], np.int32)
    for step, n_new in enumerate((np.array([1, 1, 1, 1, 1, 1]), np.array([7, 0, 40, 3, 1, 2]),
                                  np.array([1, 1, 1, 1, 1, 1]))):
        print(f"[qkv] step {step}", flush=True)
        _run(cache, st, 0, pos, n_new, hq, hkv, D, is_global, with_v, q_bf16, rng)
        _state_match(cache, st)
        pos = pos + n_new.astype(np.int32)
    cache.free()


def test_append_qkv_ring_in_place_q_and_out_of_blocks(gpu):
    # Ring pools (sliding layers' default mode), Q normalised in place (q_out aliases q),
    # and a paged call that runs out of blocks: Q is still produced, no K/V row written.
    print("[qkv] ring / in place / out of blocks", flush=True)
    rng = np.random.default_rng(77)
    hq, hkv, D, ring = 16, 8, 256, 1032
    B = 3
    cache = PagedKVCache([LayerSpec(hq, hkv, D, window=1024, ring_size=ring)], block_size=16,
                         num_blocks=8, max_seqs=B, max_blocks_per_seq=8, num_kv_slots=4)
    cache.admit(range(B))
    rs = O.RingState(1, hkv * D, ring, 4)
    pos = np.array([1030, 0, 70], np.int32)
    n_new = np.array([5, 1100, 2])  # sequence 1 writes more than the ring holds
    _run(cache, rs, 0, pos, n_new, hq, hkv, D, False, True, False, rng,
         slots=cache.kv_slot_of.copy(), q_in_place=True)
    cache.free()
    # out of blocks: 2 free blocks, sequence 0 needs 3
    cache = PagedKVCache([LayerSpec(hq, hkv, D)], block_size=16, num_blocks=2, max_seqs=2,
                         max_blocks_per_seq=8)
    st = O.CacheState(1, hkv * D, 16, 2, 2, 8)
    pos = np.array([0, 0], np.int32)
    n_new = np.array([40, 3])
    q_out, _ = _run(cache, st, 0, pos, n_new, hq, hkv, D, False, True, False, rng)
    assert list(cache.status.numpy()) == [lib.PKV_SEQ_OUT_OF_BLOCKS, lib.PKV_SEQ_OUT_OF_BLOCKS]
    assert np.all(np.isfinite(q_out.numpy()))
    _state_match(cache, st)
    assert not cache.k_pools[0].numpy().any() and not cache.v_pools[0].numpy().any()
    cache.free()


def test_append_qkv_chains_into_prefill(gpu):
    # Producer step for a 2 x 300-token chunk over prefixes (bf16 pools, bf16 Q), then
    # pkv_prefill on what it wrote. The producer's values are checked against the oracle
    # inside _run; the attention is checked as the north star's bf16 rule states it, with
    # the oracle run on the same bf16 values the GPU attended (its pools and Q).
    print("[qkv] chain into prefill", flush=True)
    rng = np.random.default_rng(5)
    hq, hkv, D, bs = 16, 8, 256, 16
    B, nb, stride = 2, 160, 80
    spec = LayerSpec(hq, hkv, D, window=0, kv_dtype=BF16)
    cache = PagedKVCache([spec], block_size=bs, num_blocks=nb, max_seqs=B,
                         max_blocks_per_seq=stride, scale=0.0625)
    st = O.CacheState(1, hkv * D, bs, nb, B, stride, dtype=np.uint16)
    zeros = np.zeros(B, np.int32)
    prefix = np.array([37, 500], np.int32)
    _run(cache, st, 0, zeros, prefix.astype(np.int64), hq, hkv, D, False, True, True, rng)
    chunk = np.array([300, 300])
    q_out, tok_off = _run(cache, st, 0, prefix, chunk, hq, hkv, D, False, True, True, rng)
    _state_match(cache, st)
    rows = int(tok_off[-1])
    out = hip.DeviceArray((rows, hq, D), np.float32)
    cache.prefill(0, q_out, prefix, tok_off, 300, out, batch=B)
    got = out.numpy()
    qb = O.bf16_to_f32(q_out.numpy()).reshape(rows, hq, D)
    k_gpu = cache.k_pools[0].numpy().reshape(-1)
    v_gpu = cache.v_pools[0].numpy().reshape(-1)
    for s in range(B):
        r0 = int(tok_off[s])
        qs = qb[r0:r0 + 300].reshape(1, 300, hq, D)
        ref = O.attend(qs, k_gpu, v_gpu, st.tables[s:s + 1],
                       st.table_lens[s:s + 1], prefix[s:s + 1], 300, hq, hkv, D, bs, 0,
                       scale=0.0625, nthreads=O.max_threads(), par=2)
        parity.check(got[r0:r0 + 300].reshape(ref.shape), ref, bf16=True, what=f"seq {s}")
    cache.free()
