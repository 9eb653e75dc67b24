"""CPU checks that pin the oracle's LSA sparse attention (pkvo_lsa_sparse_paged_attention,
pkvo_attend_sparse / _f64) and key-list expansion (pkvo_lsa_expand_buckets), and the
host-side lsa_expand_buckets of the product against it: the reference's own dense
equivalence test (test_lsa.mojo:136-198) plus closed forms."""
import numpy as np
import pytest

import pkv
from oracle import oracle as O
from tests.refcase import BLOCK_SIZE, CAPACITY, Fixture


def test_sparse_attention_dense_equivalence():
    # test_lsa.mojo:136-198: 16 q / 2 kv heads, head_dim 512, 32 tokens in blocks [0, 1];
    # q = (i % 13) * 0.01, k = (i % 17) * 0.01, v = (i % 19) * 0.01; sparse attention over
    # all 32 keys is bit-exact with dense paged_attention_layer at pos 31.
    heads, kv_heads, D, n = 16, 2, 512, 32
    kvs = kv_heads * D
    q = ((np.arange(heads * D) % 13).astype(np.float64) * 0.01).astype(np.float32)
    k = ((np.arange(n * kvs) % 17).astype(np.float64) * 0.01).astype(np.float32)
    v = ((np.arange(n * kvs) % 19).astype(np.float64) * 0.01).astype(np.float32)
    table = [0, 1]
    dense = O.paged_attention_layer(q, k, v, table, 16, n - 1, heads, kv_heads, D, 0)
    sparse = O.lsa_sparse_paged_attention(q, k, v, table, 16, list(range(n)), heads, kv_heads, D)
    np.testing.assert_array_equal(sparse, dense)


@pytest.mark.parametrize("nthreads", [1, 8])
def test_sparse_over_the_window_equals_windowed_dense(nthreads):
    fx = Fixture(16, 8, 256, seed=31, k_scale=0.25)
    for pos, window in ((0, 16), (100, 64), (1500, 1024), (CAPACITY - 1, 300)):
        ws = O.window_start(pos, window)
        dense = fx.run_new(pos, window, nthreads=nthreads)
        sparse = O.lsa_sparse_paged_attention(fx.q, fx.k_pool, fx.v_pool, fx.table, BLOCK_SIZE,
                                              list(range(ws, pos + 1)), 16, 8, 256,
                                              nthreads=nthreads)
        np.testing.assert_array_equal(sparse, dense, err_msg=f"pos={pos} window={window}")


def test_sparse_empty_list_gives_zeros_and_f64_agrees():
    fx = Fixture(16, 8, 256, seed=32, k_scale=0.25)
    out = O.lsa_sparse_paged_attention(fx.q, fx.k_pool, fx.v_pool, fx.table, BLOCK_SIZE, [],
                                       16, 8, 256)
    assert not out.any()
    rng = np.random.default_rng(0)
    tables = fx.table.astype(np.int32).reshape(1, -1)
    keys = rng.choice(CAPACITY, 700, replace=False).astype(np.int32)
    off = np.array([0, 700], np.int32)
    got = O.attend_sparse(fx.q.reshape(1, 16, 256), fx.k_pool, fx.v_pool, tables, keys, off, 16,
                          8, 256, BLOCK_SIZE)
    exact = O.attend_sparse_f64(fx.q.reshape(1, 16, 256), fx.k_pool, fx.v_pool, tables, keys,
                                off, 16, 8, 256, BLOCK_SIZE)
    assert O.max_rel_err(got, exact) < 1e-4
    # the float64 path over a key list equals the float64 path over the same range
    rng_keys = np.arange(200, 901, dtype=np.int32)
    e_list = O.attend_sparse_f64(fx.q.reshape(1, 16, 256), fx.k_pool, fx.v_pool, tables,
                                 rng_keys, np.array([0, rng_keys.size], np.int32), 16, 8, 256,
                                 BLOCK_SIZE)
    e_range = O.attention_f64(fx.q, fx.k_pool, fx.v_pool, fx.table, BLOCK_SIZE, 900, 200, 16, 8,
                              256)
    np.testing.assert_array_equal(e_list.reshape(-1), e_range)
    # key order does not change the set attended (fp32 rounding aside)
    perm = O.attend_sparse(fx.q.reshape(1, 16, 256), fx.k_pool, fx.v_pool, tables,
                           keys[::-1].copy(), off, 16, 8, 256, BLOCK_SIZE)
    assert O.max_rel_err(perm, got) < 1e-4


def _buckets(rng, nb, cap, pos):
    sizes = rng.integers(0, cap + 1, nb)
    members = np.zeros((nb, cap), np.int64)
    for b in range(nb):
        members[b, : sizes[b]] = rng.choice(pos + 1, sizes[b], replace=False)
    return sizes, members


@pytest.mark.parametrize("seed", range(6))
def test_expand_buckets_host_matches_oracle_and_its_definition(seed):
    rng = np.random.default_rng(seed)
    pos = int(rng.integers(0, 3000))
    nb, cap = 24, 40
    sizes, members = _buckets(rng, nb, cap, pos)
    picked = rng.choice(nb, int(rng.integers(0, 8)), replace=False)
    top_k, sinks, window = int(rng.integers(1, 100)), int(rng.integers(0, 8)), int(rng.integers(1, 600))
    want = O.lsa_expand_buckets(picked, sizes, members, pos, top_k, sinks, window)
    got = pkv.lsa_expand_buckets(picked, sizes, members, pos, top_k, sinks, window)
    np.testing.assert_array_equal(got, want)
    ws = max(0, pos + 1 - window)
    n_win = pos + 1 - ws
    n_sink = min(sinks, ws, pos + 1)
    n_b = got.size - n_win - n_sink
    assert 0 <= n_b <= top_k
    np.testing.assert_array_equal(got[n_b:n_b + n_win], np.arange(ws, pos + 1))
    np.testing.assert_array_equal(got[n_b + n_win:], np.arange(n_sink))
    bucket_part = got[:n_b]
    assert np.all((bucket_part >= sinks) & (bucket_part < ws))
    # bucket members are taken in picked order, each bucket's in stored order
    flat = [int(t) for b in picked for t in members[b, : sizes[b]] if sinks <= t < ws]
    np.testing.assert_array_equal(bucket_part, flat[:n_b])
    assert n_b == min(top_k, len(flat))


def _reference_position_buckets():
    """The buckets test_lsa_reference.mojo:130-148 builds in "position" mode: 64 keys,
    bucket size 16 -> bucket b holds tokens 16b .. 16b + 15 in order (bucket cap 32)."""
    sizes = np.full(4, 16, np.int32)
    members = np.zeros((4, 32), np.int32)
    for b in range(4):
        members[b, :16] = np.arange(16 * b, 16 * b + 16)
    return sizes, members


def test_expand_buckets_reference_known_answer():
    """test_lsa_reference.mojo:150-184: picked [0, 2], position 63, top_k 10, sinks 2,
    window 4 -> the first ten members of bucket 0 past the sinks, the window, the sinks:
    [2 .. 11, 60, 61, 62, 63, 0, 1]."""
    sizes, members = _reference_position_buckets()
    want = list(range(2, 12)) + [60, 61, 62, 63, 0, 1]
    got = O.lsa_expand_buckets([0, 2], sizes, members, 63, 10, 2, 4)
    assert got.tolist() == want
    assert pkv.lsa_expand_buckets([0, 2], sizes, members, 63, 10, 2, 4).tolist() == want
