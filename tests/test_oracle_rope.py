"""CPU checks that pin the oracle's producer step (rms_norm, rms_norm_noscale, apply_rope,
apply_rope_qk, pkvo_append_qkv): the reference's own RoPE test
(test_rope_and_parallel_attn.mojo:110-165, trig-hoisted RoPE bit-exact with the scalar
per-element form), plus closed forms a dropped term, a wrong sign or a wrong pair index
would fail."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O

POSITIONS = [0, 47, 1023, 1024, 100000]  # test_rope_and_parallel_attn.mojo:120


def _pattern(n, mod, off):
    # test_rope_and_parallel_attn.mojo:125-131: Float32((i % mod) - off) * 0.05
    return ((np.arange(n) % mod - off).astype(np.float32) * np.float32(0.05)).astype(np.float32)


@pytest.mark.parametrize("p_idx", range(len(POSITIONS)))
def test_rope_trig_hoisted_equals_scalar_reference(p_idx):
    p = POSITIONS[p_idx]
    # sliding: 16 q heads, 8 kv heads, head_dim 256
    q, k = _pattern(16 * 256, 41, 20), _pattern(8 * 256, 37, 18)
    qo, ko = O.apply_rope_qk(q, k, 16, 8, 256, p, False)
    np.testing.assert_array_equal(qo, O.ref_apply_rope(q, 16, 256, p, False))
    np.testing.assert_array_equal(ko, O.ref_apply_rope(k, 8, 256, p, False))
    # global: 16 q heads, 2 kv heads, head_dim 512; apply_rope_qk and apply_rope alternate
    q, k = _pattern(16 * 512, 41, 20), _pattern(2 * 512, 37, 18)
    if p_idx % 2 == 0:
        qo, ko = O.apply_rope_qk(q, k, 16, 2, 512, p, True)
    else:
        qo, ko = O.apply_rope(q, 16, 512, p, True), O.apply_rope(k, 2, 512, p, True)
    np.testing.assert_array_equal(qo, O.ref_apply_rope(q, 16, 512, p, True))
    np.testing.assert_array_equal(ko, O.ref_apply_rope(k, 2, 512, p, True))


def test_rope_position_zero_is_identity_and_global_tail_untouched():
    rng = np.random.default_rng(1)
    v = rng.standard_normal(4 * 256, dtype=np.float32)
    np.testing.assert_array_equal(O.apply_rope(v, 4, 256, 0, False), v)
    g = rng.standard_normal(2 * 512, dtype=np.float32)
    out = O.apply_rope(g, 2, 512, 777, True).reshape(2, 512)
    gi = g.reshape(2, 512)
    # only pairs (i, i + 256) with i < 64 rotate on global layers
    np.testing.assert_array_equal(out[:, 64:256], gi[:, 64:256])
    np.testing.assert_array_equal(out[:, 320:], gi[:, 320:])
    assert not np.array_equal(out[:, :64], gi[:, :64])


@pytest.mark.parametrize("is_global,D", [(False, 256), (True, 512)])
def test_rope_is_a_rotation_by_position(is_global, D):
    # Pair norms are preserved, and q(p).k(p') depends only on p - p': a flipped sign on
    # one sin term or a wrong pair partner breaks both.
    rng = np.random.default_rng(2)
    q = rng.standard_normal(D, dtype=np.float32)
    k = rng.standard_normal(D, dtype=np.float32)
    half = D // 2
    for p in (5, 300, 1500):
        r = O.apply_rope(q, 1, D, p, is_global)
        n0 = q[:half].astype(np.float64) ** 2 + q[half:].astype(np.float64) ** 2
        n1 = r[:half].astype(np.float64) ** 2 + r[half:].astype(np.float64) ** 2
        np.testing.assert_allclose(n1, n0, rtol=2e-6, atol=1e-6)
    scale = float(np.linalg.norm(q) * np.linalg.norm(k))
    for p, pp, delta in ((10, 3, 200), (900, 40, 333), (64, 1000, 1)):
        d0 = float(np.dot(O.apply_rope(q, 1, D, p, is_global).astype(np.float64),
                          O.apply_rope(k, 1, D, pp, is_global)))
        d1 = float(np.dot(O.apply_rope(q, 1, D, p + delta, is_global).astype(np.float64),
                          O.apply_rope(k, 1, D, pp + delta, is_global)))
        assert abs(d0 - d1) <= 1e-4 * scale, (p, pp, delta, d0, d1)
    # and it does depend on p - p' (the rotation is not the identity)
    d_a = float(np.dot(O.apply_rope(q, 1, D, 0, is_global), O.apply_rope(k, 1, D, 0, is_global)))
    d_b = float(np.dot(O.apply_rope(q, 1, D, 7, is_global), O.apply_rope(k, 1, D, 0, is_global)))
    assert abs(d_a - d_b) > 1e-3 * scale


def test_rope_angles_first_pair_is_position_in_radians():
    # Pair 0 has frequency base^0 = 1, so (1, 0) at position p becomes (cos p, sin p).
    v = np.zeros(256, np.float32)
    v[0] = 1.0
    for p in (1, 2, 100):
        r = O.apply_rope(v, 1, 256, p, False)
        np.testing.assert_allclose([r[0], r[128]], [np.cos(p), np.sin(p)], atol=2e-6)
    # pair i rotates by p / 10000^(2i/256): check one slow pair against float64
    v = np.zeros(256, np.float32)
    v[100] = 1.0
    r = O.apply_rope(v, 1, 256, 5000, False)
    th = 5000 / 10000.0 ** (200 / 256)
    np.testing.assert_allclose([r[100], r[228]], [np.cos(th), np.sin(th)], atol=1e-5)


def test_rope_frequencies_equal_correctly_rounded_pow():
    # The GPU computes base^(2i / rope_dim) in double and rounds once to fp32; the oracle
    # (and a Mojo build through libm) use powf. They agree on every exponent in use.
    libm = ctypes.CDLL("libm.so.6")
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    for base, rope_dim, pairs in ((10000.0, 256.0, 256), (1000000.0, 512.0, 64)):
        for i in range(pairs):
            e = float(np.float32(2 * i) / np.float32(rope_dim))
            assert np.float32(libm.powf(base, e)) == np.float32(base ** e), (base, i)


def test_rms_norm_matches_float64_closed_form():
    rng = np.random.default_rng(4)
    for D in (256, 512):
        x = (rng.standard_normal(D) * 3).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6)
        np.testing.assert_allclose(O.rms_norm(x, w), want * w, rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(O.rms_norm_noscale(x), want, rtol=2e-6, atol=1e-7)
    # the epsilon matters for small vectors: mean(x^2) = 1e-6 halves the squared norm
    x = np.full(256, 1e-3, np.float32)
    np.testing.assert_allclose(O.rms_norm_noscale(x), 1e-3 / np.sqrt(2e-6), rtol=1e-5)


def _qkv_case(rng, B, n_new, hq, hkv, D, with_v):
    tok_off = O.ragged_tok_off(n_new)
    rows = int(tok_off[-1])
    q = rng.standard_normal((rows, hq * D), dtype=np.float32) * 2
    k = rng.standard_normal((rows, hkv * D), dtype=np.float32) * 2
    v = rng.standard_normal((rows, hkv * D), dtype=np.float32) if with_v else None
    qw = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    kw = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    return tok_off, rows, q, k, v, qw, kw


@pytest.mark.parametrize("is_global,hq,hkv,D,with_v", [(False, 16, 8, 256, True),
                                                       (True, 16, 2, 512, False)])
def test_append_qkv_is_norm_then_rope_then_append(is_global, hq, hkv, D, with_v):
    # The fused oracle equals the engine's sequence done step by step with the restated
    # functions: per-head norms, apply_rope_qk at the token's position, then the append of
    # the processed rows; v=None means V := K as read (before the norms).
    rng = np.random.default_rng(9)
    B = 3
    n_new = np.array([5, 1, 17])
    pos = np.array([14, 0, 31], np.int32)
    tok_off, rows, q, k, v, qw, kw = _qkv_case(rng, B, n_new, hq, hkv, D, with_v)
    kvs = hkv * D
    fused = O.CacheState(1, kvs, 16, 12, B, 8)
    st, q_out = O.append_qkv(fused, 0, pos, tok_off, q, k, v, qw, kw, 20, hq, hkv, D, is_global)
    assert np.all(st == 0)
    step = O.CacheState(1, kvs, 16, 12, B, 8)
    qn = np.empty_like(q)
    kn = np.empty_like(k)
    vn = np.empty_like(k)
    vsrc = k if v is None else v
    for s in range(B):
        for b in range(int(n_new[s])):
            r = int(tok_off[s]) + b
            qh = np.concatenate([O.rms_norm(q[r, h * D:(h + 1) * D], qw) for h in range(hq)])
            kh = np.concatenate([O.rms_norm(k[r, h * D:(h + 1) * D], kw) for h in range(hkv)])
            vn[r] = np.concatenate([O.rms_norm_noscale(vsrc[r, h * D:(h + 1) * D])
                                    for h in range(hkv)])
            qn[r], kn[r] = O.apply_rope_qk(qh, kh, hq, hkv, D, int(pos[s]) + b, is_global)
    assert np.all(step.append(0, pos, tok_off, kn, vn, 20) == 0)
    np.testing.assert_array_equal(q_out, qn)
    np.testing.assert_array_equal(fused.k_pools[0], step.k_pools[0])
    np.testing.assert_array_equal(fused.v_pools[0], step.v_pools[0])
    np.testing.assert_array_equal(fused.tables, step.tables)
    np.testing.assert_array_equal(fused.free_list, step.free_list)


@pytest.mark.parametrize("is_global,hq,hkv,D", [(False, 16, 8, 256), (True, 16, 2, 512)])
def test_producer_f64_agrees_with_fp32_oracle(is_global, hq, hkv, D):
    # The float64 producer evaluates the same formula: it differs from the fp32 oracle only
    # by fp32 rounding of terms of magnitude <= ~10, and V := K when v is None.
    rng = np.random.default_rng(12)
    n_new = np.array([3, 0, 9])
    pos = np.array([0, 5, 100000], np.int32)
    tok_off, rows, q, k, v, qw, kw = _qkv_case(rng, 3, n_new, hq, hkv, D, not is_global)
    st = O.CacheState(1, hkv * D, 16, 8, 3, 6300)
    st.table_lens[2] = 100000 // 16
    status, q32 = O.append_qkv(st, 0, pos, tok_off, q, k, v, qw, kw, 9, hq, hkv, D, is_global)
    assert np.all(status == 0)
    q64, k64, v64 = O.producer_f64(pos, tok_off, q, k, v, qw, kw, 9, hq, hkv, D, is_global)
    np.testing.assert_allclose(q64, q32, rtol=0, atol=2e-5)
    # the pool rows of sequence 2 (one fresh block) hold its 9 tokens
    kvs = hkv * D
    blk = int(st.tables[2, 100000 // 16])
    k_rows = st.k_pools[0].reshape(-1, kvs)[blk * 16: blk * 16 + 9]
    v_rows = st.v_pools[0].reshape(-1, kvs)[blk * 16: blk * 16 + 9]
    np.testing.assert_allclose(k64[3:12], k_rows, rtol=0, atol=2e-5)
    np.testing.assert_allclose(v64[3:12], v_rows, rtol=0, atol=2e-5)
