"""CPU checks that pin the oracle's attention (oracle/pkv_oracle.c) -- the reference's
own test_attention.mojo / test_rope_and_parallel_attn.mojo checks, plus closed forms."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.refcase import BLOCK_SIZE, CAPACITY, Fixture


def test_window_start():
    # Known answers, test_attention.mojo:272-284.
    assert O.window_start(0, 0) == 0
    assert O.window_start(5000, 0) == 0
    assert O.window_start(5000, -1) == 0
    assert O.window_start(0, 1024) == 0
    assert O.window_start(1022, 1024) == 0
    assert O.window_start(1023, 1024) == 0
    assert O.window_start(1024, 1024) == 1
    assert O.window_start(2047, 1024) == 1024
    assert O.window_start(10, 1) == 10


def test_ring_row():
    # Known answers, test_attention.mojo:624-631.
    assert O.ring_row(0, 1024, 0) == 0
    assert O.ring_row(0, 1024, 1023) == 1023
    assert O.ring_row(0, 1024, 1024) == 0
    assert O.ring_row(1, 1024, 0) == 1024
    assert O.ring_row(1, 1024, 2049) == 1024 + 1
    assert O.ring_row(3, 100, 250) == 350


def test_lcg_reproduces_reference_construction():
    # test_attention.mojo:27-37: state = seed*A + C, then per draw state = state*A + C and
    # ((state >> 40) & 0xFFFFFF) / 2^23 - 1. Recomputed here with Python integers.
    A, C, M = 6364136223846793005, 1442695040888963407, (1 << 64) - 1
    st = (42 * A + C) & M
    want = []
    for _ in range(16):
        st = (st * A + C) & M
        want.append(np.float32(((st >> 40) & 0xFFFFFF) / float(0x800000) - 1.0))
    got = O.Lcg(42).fill(16, 1.0)
    np.testing.assert_array_equal(got, np.array(want, np.float32))
    assert np.all(got >= -1.0) and np.all(got < 1.0)


@pytest.mark.parametrize("geom", [(16, 2, 512), (16, 8, 256)], ids=["global", "sliding"])
def test_full_bit_exact(geom):
    # test_attention.mojo:287-296: the refactored kernel is bit-exact with the legacy loop.
    fx = Fixture(*geom, seed=42, k_scale=0.25)
    for p in [0, 1, 15, 16, 17, 99, 100, 101, 777, 1023, 1024, CAPACITY - 1]:
        np.testing.assert_array_equal(fx.run_new(p, 0), fx.run_legacy(p), err_msg=f"pos={p}")


def test_window_is_noop_when_short():
    # test_attention.mojo:299-308
    fx = Fixture(16, 8, 256, seed=7, k_scale=0.25)
    for p in [0, 5, 512, 1022, 1023]:
        np.testing.assert_array_equal(fx.run_new(p, 1024), fx.run_legacy(p))


def test_window_matches_reference():
    # test_attention.mojo:311-321 (f64 oracle, 1e-4)
    fx = Fixture(16, 8, 256, seed=99, k_scale=0.25)
    for p in [1024, 1025, 1500, 2047, CAPACITY - 1]:
        err = O.max_rel_err(fx.run_new(p, 1024), fx.run_reference(p, p - 1023))
        assert err < 1e-4, (p, err)


def test_window_boundary_is_exact():
    # test_attention.mojo:324-365
    fx = Fixture(16, 8, 256, seed=3, k_scale=0.01)
    pos = 2000
    fx.plant(pos - 1024)  # just outside
    out = fx.run_new(pos, 1024)
    assert np.all(np.abs(out) < 10.0)
    # Copy the planted key to the inside edge (the outside copy stays).
    ri, ro = fx.row_of(pos - 1023), fx.row_of(pos - 1024)
    fx.k_pool[ri:ri + fx.kv_stride] = fx.k_pool[ro:ro + fx.kv_stride]
    fx.v_pool[ri:ri + fx.kv_stride] = 1000.0
    out = fx.run_new(pos, 1024)
    assert np.all(out > 900.0)


def test_large_scores_stable():
    # test_attention.mojo:368-380 (K x4, no softmax scale)
    fx = Fixture(16, 2, 512, seed=11, k_scale=4.0)
    for p in [0, 300, CAPACITY - 1]:
        out = fx.run_new(p, 0)
        np.testing.assert_array_equal(out, fx.run_legacy(p))
        assert np.all(np.isfinite(out)) and np.all(np.abs(out) < 1e30)


def test_tight_scratch_contract():
    # test_attention.mojo:383-437: scratch sized exactly (Hq*n, n) + canaries.
    guard, canary = 64, np.float32(-12345.678)
    for geom in [(16, 2, 512), (16, 8, 256), (8, 8, 64)]:
        fx = Fixture(*geom, seed=5, k_scale=0.25)
        for p in [0, 1, 1023, 1024, 1500, CAPACITY - 1]:
            for w in [0, 1, 7, 1024]:
                n = p + 1 - O.window_start(p, w)
                scores = np.full(fx.heads * n + guard, canary, np.float32)
                rows = np.full(n + guard, -777, np.int64)
                out = np.full(fx.heads * fx.head_dim + guard, canary, np.float32)
                O.paged_attention_layer(fx.q, fx.k_pool, fx.v_pool, fx.table, BLOCK_SIZE, p,
                                        fx.heads, fx.kv_heads, fx.head_dim, w, scores, rows, out)
                assert np.all(scores[fx.heads * n:] == canary)
                assert np.all(rows[n:] == -777)
                assert np.all(out[fx.heads * fx.head_dim:] == canary)


def test_ratio_one_and_seeds():
    # test_attention.mojo:420-437
    for seed in [1, 2]:
        fx = Fixture(8, 8, 64, seed=seed, k_scale=0.5)
        for p in [0, 33, CAPACITY - 1]:
            np.testing.assert_array_equal(fx.run_new(p, 0), fx.run_legacy(p))
    fx2 = Fixture(16, 2, 512, seed=1234, k_scale=0.25)
    for p in [5, 640, CAPACITY - 1]:
        np.testing.assert_array_equal(fx2.run_new(p, 0), fx2.run_legacy(p))


def test_window_block_aligned_edge():
    # test_attention.mojo:440-497
    fx = Fixture(16, 8, 256, seed=21, k_scale=0.01)
    pos = 1024 + 16 * 3 + 1023
    start = O.window_start(pos, 1024)
    assert start % BLOCK_SIZE == 0
    fx.plant(start - 1)
    assert np.all(np.abs(fx.run_new(pos, 1024)) < 10.0)
    fx.plant(start)
    assert np.all(fx.run_new(pos, 1024) > 900.0)
    fx3 = Fixture(16, 8, 256, seed=22, k_scale=0.01)
    fx3.plant(1777)
    assert np.all(fx3.run_new(1777, 1024) > 900.0)


def test_parallel_matches_serial():
    # test_rope_and_parallel_attn.mojo:199-261: head-pair tasks on threads are bit-exact
    # with the serial loop, including the odd-ratio (12q/4kv) pair + single-head tail.
    fx = Fixture(16, 8, 256, seed=9, k_scale=0.25)
    for p in [0, 62, 63, 511, 2047]:
        np.testing.assert_array_equal(fx.run_new(p, 1024, nthreads=8), fx.run_new(p, 1024))
    fx12 = Fixture(12, 4, 256, seed=9, k_scale=0.25)
    out = fx12.run_new(127, 1024, nthreads=8)
    ref = fx12.run_reference(127, 0)
    assert O.max_rel_err(out, ref) < 1e-4


def test_single_key_returns_value_row_exactly():
    # n = 1: softmax gives 1 / (1 + 1e-10) == 1.0f, so out = V row bit-exactly.
    fx = Fixture(16, 8, 256, seed=4, k_scale=1.0)
    out = fx.run_new(777, 1)
    r = fx.row_of(777)
    for h in range(16):
        g = h // 2
        np.testing.assert_array_equal(out[h * 256:(h + 1) * 256],
                                      fx.v_pool[r + g * 256:r + (g + 1) * 256])


def test_identical_keys_give_mean_of_values():
    # Equal scores -> uniform weights -> mean of V (closed form, f64 within 1e-5).
    fx = Fixture(16, 8, 256, seed=6, k_scale=1.0)
    pos = 100
    k0 = fx.k_pool[fx.row_of(0):fx.row_of(0) + fx.kv_stride].copy()
    for t in range(pos + 1):
        fx.k_pool[fx.row_of(t):fx.row_of(t) + fx.kv_stride] = k0
    out = fx.run_new(pos, 0).astype(np.float64)
    vs = np.stack([fx.v_pool[fx.row_of(t):fx.row_of(t) + fx.kv_stride] for t in range(pos + 1)])
    mean = vs.astype(np.float64).mean(axis=0)
    for h in range(16):
        g = h // 2
        np.testing.assert_allclose(out[h * 256:(h + 1) * 256], mean[g * 256:(g + 1) * 256],
                                   rtol=0, atol=1e-5)


def test_bf16_pool_is_fp32_pool_upcast():
    # A bf16 pool is read by exact upcast: identical bits to the fp32 run on upcast values.
    fx = Fixture(16, 8, 256, seed=8, k_scale=0.25)
    kb, vb = O.to_bf16(fx.k_pool), O.to_bf16(fx.v_pool)
    ku, vu = O.bf16_to_f32(kb), O.bf16_to_f32(vb)
    for p in [0, 700, 2000]:
        a = O.paged_attention_layer(fx.q, kb, vb, fx.table, BLOCK_SIZE, p, 16, 8, 256, 1024)
        b = O.paged_attention_layer(fx.q, ku, vu, fx.table, BLOCK_SIZE, p, 16, 8, 256, 1024)
        np.testing.assert_array_equal(a, b)


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -2.5, 3.0e38, np.inf, 0.0],
                 np.float32)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 1.5*2^-8 rounds up to 1 + 2^-7.
    want = np.array([1.0, 1.0, 1.0078125, 1.0078125, -2.5], np.float32)
    got = O.bf16_to_f32(O.to_bf16(x))
    np.testing.assert_array_equal(got[:5], want)
    assert got[6] == np.inf and got[7] == 0.0


def test_power_of_two_scale_is_exact():
    # BASELINE configs use scale 1/sqrt(256) = 2^-4; pre-scaling q is exact.
    fx = Fixture(16, 8, 256, seed=12, k_scale=1.0)
    tables = fx.table[None, :].astype(np.int32)
    lens = np.array([len(fx.table)], np.int32)
    q = fx.q.reshape(1, 1, 16, 256)
    a = O.attend(q, fx.k_pool, fx.v_pool, tables, lens, np.array([900], np.int32), 1, 16, 8, 256,
                 BLOCK_SIZE, 0, scale=0.0625)
    b = O.attend(q * np.float32(0.0625), fx.k_pool, fx.v_pool, tables, lens,
                 np.array([900], np.int32), 1, 16, 8, 256, BLOCK_SIZE, 0)
    np.testing.assert_array_equal(a, b)


def test_attend_matches_per_token_calls_and_inactive_is_zero():
    fx = Fixture(16, 8, 256, seed=13, k_scale=0.25)
    tables = np.stack([fx.table, fx.table[::-1]]).astype(np.int32)
    lens = np.array([160, 160], np.int32)
    rng = np.random.default_rng(0)
    q = rng.standard_normal((2, 3, 16, 256)).astype(np.float32)
    out = O.attend(q, fx.k_pool, fx.v_pool, tables, lens, np.array([500, -1], np.int32), 3, 16,
                   8, 256, BLOCK_SIZE, 1024)
    for j in range(3):
        ref = O.paged_attention_layer(q[0, j].reshape(-1), fx.k_pool, fx.v_pool, tables[0],
                                      BLOCK_SIZE, 500 + j, 16, 8, 256, 1024)
        np.testing.assert_array_equal(out[0, j].reshape(-1), ref)
    assert np.all(out[1] == 0.0)


def test_batched_f64_oracle_agrees_with_per_token_f64():
    fx = Fixture(16, 8, 256, seed=14, k_scale=0.25)
    tables = fx.table[None, :].astype(np.int32)
    q = np.random.default_rng(1).standard_normal((1, 3, 16, 256)).astype(np.float32)
    ex = O.attend_f64(q, fx.k_pool, fx.v_pool, tables, np.array([1500], np.int32), 3, 16, 8, 256,
                      BLOCK_SIZE, 1024, scale=0.0625)
    for j in range(3):
        p = 1500 + j
        want = O.attention_f64(q[0, j].reshape(-1) * np.float32(0.0625), fx.k_pool, fx.v_pool,
                               fx.table, BLOCK_SIZE, p, p - 1023, 16, 8, 256)
        np.testing.assert_array_equal(ex[0, j].reshape(-1), want)
    r32 = O.attend(q, fx.k_pool, fx.v_pool, tables, np.array([160], np.int32),
                   np.array([1500], np.int32), 3, 16, 8, 256, BLOCK_SIZE, 1024, scale=0.0625)
    assert O.max_rel_err(r32, ex) < 1e-4


@pytest.mark.parametrize("geom", [(16, 8, 256), (16, 2, 512), (6, 3, 64), (5, 5, 64)],
                         ids=["16q8kv", "16q2kv", "ratio2-odd-pairs", "odd-heads"])
def test_every_parallel_mode_gives_the_same_bits(geom):
    """par 0 (reference-faithful: head-pair tasks per call), 1 (sequences over threads),
    2 ((sequence, query) items) and 3 (every core on (sequence, query, head pair) items,
    the batched CPU baseline) compute each head with the same arithmetic: identical bits,
    including calls below the head-pair condition (n < 64, odd ratio or head count),
    windows and an inactive sequence."""
    hq, hkv, d = geom
    fx = Fixture(hq, hkv, d, seed=21, k_scale=0.25)
    tables = np.stack([fx.table, fx.table[::-1], fx.table, fx.table[::-1]]).astype(np.int32)
    lens = np.full(4, 160, np.int32)
    pos = np.array([700, 30, -1, 2000], np.int32)  # 30: n < 64 -> the serial path
    q = np.random.default_rng(2).standard_normal((4, 2, hq, d)).astype(np.float32)
    outs = [O.attend(q, fx.k_pool, fx.v_pool, tables, lens, pos, 2, hq, hkv, d, BLOCK_SIZE, w,
                     scale=0.0625, nthreads=4, par=par)
            for w in (0, 512) for par in (0, 1, 2, 3)]
    for i in range(1, 4):
        np.testing.assert_array_equal(outs[i], outs[0])
        np.testing.assert_array_equal(outs[4 + i], outs[4])
    assert np.all(outs[0][2] == 0.0)
