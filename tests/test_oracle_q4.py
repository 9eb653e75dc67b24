"""CPU checks that pin the oracle's Q4_0 restatements (quantize_fp32_to_q4_0,
q4_matmul_vec): the reference's own scalar-oracle test (test_q4_4row_tiling.mojo:106-136)
restated, plus closed forms of the block format."""
import numpy as np

from oracle import oracle as O


def _reference_patterns(c_in, c_out):
    # test_q4_4row_tiling.mojo:119-124
    x = ((np.arange(c_in) % 31 - 15).astype(np.float32) * np.float32(0.02)).astype(np.float32)
    packed = ((np.arange(c_out * (c_in // 2), dtype=np.int64) * 13 + 7) & 255).astype(np.uint8)
    scales = (((np.arange(c_out * (c_in // 32)) % 19) + 1).astype(np.float32)
              * np.float32(0.002)).astype(np.float32)
    return x, packed.reshape(c_out, -1), scales.reshape(c_out, -1)


def test_vectorized_matches_scalar_oracle_on_reference_patterns():
    # test_q4_4row_tiling.mojo:126-136: c_in 2816, the first 67 rows, max |diff| <= 1e-4.
    x, packed, scales = _reference_patterns(2816, 67)
    vec = O.q4_matmul_vec(packed, scales, x)
    sca = O.scalar_q4(packed, scales, x)
    assert np.max(np.abs(vec - sca)) <= 1e-4
    exact = O.q4_matmul_f64(packed, scales, x)
    assert np.max(np.abs(vec - exact)) <= 1e-4


def test_exact_when_every_product_and_sum_is_representable():
    # Power-of-two scales and small integer inputs keep every fp32 product and partial sum
    # exact, so both restatements equal the float64 product bit for bit.
    rng = np.random.default_rng(1)
    c_in, c_out = 256, 40
    packed = rng.integers(0, 256, (c_out, c_in // 2)).astype(np.uint8)
    scales = (2.0 ** rng.integers(-3, 3, (c_out, c_in // 32))).astype(np.float32)
    x = rng.integers(-4, 5, c_in).astype(np.float32)
    exact = O.q4_matmul_f64(packed, scales, x)
    np.testing.assert_array_equal(O.q4_matmul_vec(packed, scales, x), exact.astype(np.float32))
    np.testing.assert_array_equal(O.scalar_q4(packed, scales, x), exact.astype(np.float32))


def test_nibble_order_and_offset():
    # Byte j of a block holds element 2j (low nibble) and 2j + 1 (high nibble), offset 8:
    # a one-hot x picks exactly one dequantized weight.
    packed = np.zeros((1, 16), np.uint8)
    packed[0, 3] = (7 + 8) | ((-8 + 8) << 4)  # element 6 = 7, element 7 = -8
    scales = np.array([[0.5]], np.float32)
    for k, want in ((6, 3.5), (7, -4.0), (0, -4.0)):  # untouched bytes hold 0 -> -8
        x = np.zeros(32, np.float32)
        x[k] = 1.0
        assert O.q4_matmul_vec(packed, scales, x)[0] == np.float32(want)


def test_quantize_block_format():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((8, 128)) * 3).astype(np.float32)
    packed, scales = O.quantize_q4_0(w)
    blocks = w.reshape(8, 4, 32)
    np.testing.assert_allclose(scales, np.maximum(np.abs(blocks).max(-1) / 7, 1e-5), rtol=1e-6)
    lo = (packed & 15).astype(np.int64) - 8
    hi = (packed >> 4).astype(np.int64) - 8
    q = np.empty((8, 128), np.int64)
    q[:, 0::2], q[:, 1::2] = lo, hi
    deq = q.reshape(8, 4, 32) * scales[..., None]
    # round to nearest: every value within half a step; the block's largest value is +-7
    assert np.all(np.abs(deq - blocks) <= scales[..., None] * (0.5 + 1e-6))
    amax = np.abs(blocks).argmax(-1)
    assert np.all(np.abs(np.take_along_axis(q.reshape(8, 4, 32), amax[..., None], -1)) == 7)
    # an all-zero block takes the 1e-5 floor and quantizes to the offset
    packed0, scales0 = O.quantize_q4_0(np.zeros((1, 32), np.float32))
    assert scales0[0, 0] == np.float32(1e-5) and np.all(packed0 == 0x88)
