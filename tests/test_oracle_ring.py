"""CPU checks that pin the oracle's ring-pool path (pkvo_ring_append, pkvo_attend /
pkvo_attend_f64 with ring_size > 0): the reference's own ring tests
(test_attention.mojo:500-614) restated, plus the write-order semantics of a batched
ring append."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.refcase import BLOCK_SIZE, CAPACITY, Fixture


def test_ring_matches_paged():
    # test_attention.mojo:500-548: the attended window placed in a poisoned ring gives
    # bit-identical output to paged addressing; evicted rows are never read.
    heads, kv_heads, head_dim, window = 16, 8, 256, 1024
    kv_stride = kv_heads * head_dim
    ring_size, num_slots = 1024 + 64, 3
    fx = Fixture(heads, kv_heads, head_dim, seed=77, k_scale=0.25)
    k_pool = fx.k_pool.reshape(-1, kv_stride)
    v_pool = fx.v_pool.reshape(-1, kv_stride)
    for slot in (0, 2):
        ring_base = slot * ring_size
        for pos in (0, 1, 1023, 1024, 1087, 1088, 1089, 2000, CAPACITY - 1):
            ring_k = np.full((num_slots * ring_size, kv_stride), 9999.0, np.float32)
            ring_v = np.full((num_slots * ring_size, kv_stride), -9999.0, np.float32)
            for t in range(O.window_start(pos, window), pos + 1):
                src = fx.row_of(t) // kv_stride
                ring_k[ring_base + t % ring_size] = k_pool[src]
                ring_v[ring_base + t % ring_size] = v_pool[src]
            paged = fx.run_new(pos, window)
            ring = O.paged_attention_layer(fx.q, ring_k.reshape(-1), ring_v.reshape(-1), [],
                                           BLOCK_SIZE, pos, heads, kv_heads, head_dim, window,
                                           ring_size=ring_size, ring_base=ring_base)
            np.testing.assert_array_equal(ring, paged, err_msg=f"slot={slot} pos={pos}")


def test_ring_interleaved_writes():
    # test_attention.mojo:565-614: two sequences (slots 0 and 1) decode in lockstep, each
    # writing its K/V at ring_row(slot, ring_size, pos) -- here through the batched ring
    # append -- then attending; every sampled step is bit-identical to paged attention
    # over that sequence's history.
    heads, kv_heads, head_dim, window = 16, 8, 256, 1024
    kv_stride = kv_heads * head_dim
    ring_size = window
    fa = Fixture(heads, kv_heads, head_dim, seed=301, k_scale=0.25)
    fb = Fixture(heads, kv_heads, head_dim, seed=302, k_scale=0.25)
    rs = O.RingState(1, kv_stride, ring_size, 2)
    rs.k_pools[0][:] = 9999.0
    rs.v_pools[0][:] = -9999.0
    slots = np.array([0, 1], np.int32)
    tok_off = O.dense_tok_off(2, 1)
    checked = 0
    for pos in range(min(2600, CAPACITY)):
        rows = [fa.row_of(pos), fb.row_of(pos)]
        k_new = np.stack([fa.k_pool[rows[0]:rows[0] + kv_stride],
                          fb.k_pool[rows[1]:rows[1] + kv_stride]])
        v_new = np.stack([fa.v_pool[rows[0]:rows[0] + kv_stride],
                          fb.v_pool[rows[1]:rows[1] + kv_stride]])
        st = rs.append(0, slots, [pos, pos], tok_off, k_new, v_new, 1)
        assert np.all(st == 0)
        near_wrap = (pos % ring_size) < 3 or (pos % ring_size) > ring_size - 3
        if near_wrap or pos % 97 == 0 or pos == CAPACITY - 1:
            for slot, fx in ((0, fa), (1, fb)):
                ring = O.paged_attention_layer(
                    fx.q, rs.k_pools[0], rs.v_pools[0], [], BLOCK_SIZE, pos, heads, kv_heads,
                    head_dim, window, ring_size=ring_size,
                    ring_base=O.ring_row(slot, ring_size, 0))
                np.testing.assert_array_equal(ring, fx.run_new(pos, window),
                                              err_msg=f"slot={slot} pos={pos}")
                checked += 1
    assert checked > 50


def test_ring_smaller_than_window_is_rejected():
    # attention.mojo:264-266: the reference aborts when the window exceeds the ring.
    fx = Fixture(16, 8, 256, seed=5, k_scale=0.25)
    ring = np.zeros(2 * 100 * fx.kv_stride, np.float32)
    O.paged_attention_layer(fx.q, ring, ring, [], BLOCK_SIZE, 99, 16, 8, 256, 0,
                            ring_size=100, ring_base=0)
    with pytest.raises(RuntimeError):
        O.paged_attention_layer(fx.q, ring, ring, [], BLOCK_SIZE, 100, 16, 8, 256, 0,
                                ring_size=100, ring_base=0)


@pytest.mark.parametrize("dtype", [np.float32, np.uint16], ids=["f32", "bf16"])
def test_ring_append_is_serial_per_token_writes(dtype):
    # The batched ring append equals the engine's per-token copy to ring_row(kv_slot,
    # ring, p) (…batched.mojo:1996, :2625, :3111) done sequence by sequence, token by
    # token -- including a call with more new tokens than the ring holds, where the
    # later tokens overwrite the earlier ones.
    rng = np.random.default_rng(3)
    kv_stride, ring_size, num_slots = 64, 20, 4
    rs = O.RingState(1, kv_stride, ring_size, num_slots, dtype=dtype)
    ref_k = np.zeros((num_slots * ring_size, kv_stride), dtype)
    ref_v = np.zeros_like(ref_k)
    pos = np.zeros(3, np.int64)
    slots = np.array([2, 0, 3], np.int32)
    for step in range(12):
        n_new = rng.integers(0, 30, size=3)  # up to 1.5 rings in one call
        tok_off = O.ragged_tok_off(n_new)
        total = int(tok_off[-1])
        k_new = rng.integers(0, 60000, size=(max(total, 1), kv_stride)).astype(dtype)
        v_new = rng.integers(0, 60000, size=(max(total, 1), kv_stride)).astype(dtype)
        st = rs.append(0, slots, pos.astype(np.int32), tok_off, k_new, v_new, 30)
        assert np.all(st == 0)
        for s in range(3):
            for b in range(int(n_new[s])):
                r = O.ring_row(int(slots[s]), ring_size, int(pos[s]) + b)
                ref_k[r] = k_new[tok_off[s] + b]
                ref_v[r] = v_new[tok_off[s] + b]
        pos += n_new
        np.testing.assert_array_equal(rs.k_pools[0].reshape(ref_k.shape), ref_k, f"step {step}")
        np.testing.assert_array_equal(rs.v_pools[0].reshape(ref_v.shape), ref_v, f"step {step}")


def test_ring_append_bad_slot_and_args_write_nothing():
    kv_stride, ring_size = 8, 10
    rs = O.RingState(1, kv_stride, ring_size, 2)
    k_new = np.ones((6, kv_stride), np.float32)
    st = rs.append(0, [0, 5, -1, 1], [0, 0, 0, 0], [0, 1, 2, 3, 9], k_new, k_new, 4)
    # slot 5 and -1 lie outside the pool (-3); rows 3..9 exceed total_rows (-5)
    assert list(st) == [0, -3, -3, -5]
    assert np.count_nonzero(rs.k_pools[0]) == kv_stride  # only sequence 0's row


@pytest.mark.parametrize("q_len,window", [(1, 24), (4, 24), (3, 0)])
def test_batched_ring_attend_equals_paged_attend(q_len, window):
    # Batched oracle attention over ring pools == over paged pools holding the same keys
    # (bit-exact in fp32: the same values in the same order); the float64 oracle agrees
    # likewise through its one-row-per-block ring table.
    rng = np.random.default_rng(11)
    H, Hkv, D, bs, ring_size = 4, 2, 64, 4, 28
    kv_stride = Hkv * D
    B, nblk = 3, 40
    pos = np.array([5, 40, 23], np.int32)
    if window == 0:
        pos = np.array([5, 22, 24], np.int32)  # every sequence's keys fit the ring
    cs = O.CacheState(1, kv_stride, bs, nblk, B, 16)
    rs = O.RingState(1, kv_stride, ring_size, B + 1)
    slots = np.array([[3], [0], [2]], np.int32)
    n_tok = pos + q_len
    tok_off = O.ragged_tok_off(n_tok)
    k = rng.standard_normal((int(tok_off[-1]), kv_stride), dtype=np.float32)
    v = rng.standard_normal((int(tok_off[-1]), kv_stride), dtype=np.float32)
    zeros = np.zeros(B, np.int32)
    assert np.all(cs.append(0, zeros, tok_off, k, v, int(n_tok.max())) == 0)
    assert np.all(rs.append(0, slots[:, 0], zeros, tok_off, k, v, int(n_tok.max())) == 0)
    q = rng.standard_normal((B, q_len, H, D), dtype=np.float32)
    args = (q_len, H, Hkv, D, bs, window)
    paged = O.attend(q, cs.k_pools[0], cs.v_pools[0], cs.tables, cs.table_lens, pos, *args,
                     scale=0.125)
    ring = O.attend(q, rs.k_pools[0], rs.v_pools[0], slots, np.zeros(B, np.int32), pos, *args,
                    scale=0.125, ring_size=ring_size)
    np.testing.assert_array_equal(ring, paged)
    p64 = O.attend_f64(q, cs.k_pools[0], cs.v_pools[0], cs.tables, pos, *args, scale=0.125)
    r64 = O.attend_f64(q, rs.k_pools[0], rs.v_pools[0], slots, pos, *args, scale=0.125,
                       ring_size=ring_size)
    np.testing.assert_array_equal(r64, p64)
