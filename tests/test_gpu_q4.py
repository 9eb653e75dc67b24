"""GPU parity of the Wo projection (pkv_q4_matmul) against the oracle's restatement of
q4_matmul_vec (moe_kernels.mojo:59-163).

Tolerances. The outputs are fp32 sums of c_in terms, so the attention rule's 1e-3 floor
does not fit them. Two checks instead:
  - the reference's own acceptance test between two fp32 implementations
    (test_q4_4row_tiling.mojo:126-136): max |x - ref| <= 1e-4 on its patterns;
  - a dot-product error bound against the float64 product: per output,
    |x - exact| <= 1e-6 * sum_k |w_k x_k| (the fp32 oracle itself stays within it), which a
    bf16-rounded input (2^-9 relative) or a dropped block would fail."""
import numpy as np
import pytest

import pkv
from oracle import oracle as O
from pkv import hip

pytestmark = pytest.mark.gpu


def _dequant(packed, scales):
    lo = (packed & 15).astype(np.float64) - 8
    hi = (packed >> 4).astype(np.float64) - 8
    w = np.empty((packed.shape[0], packed.shape[1] * 2))
    w[:, 0::2], w[:, 1::2] = lo, hi
    return w * np.repeat(scales.astype(np.float64), 32, axis=1)


def _run(packed, scales, x):
    batch, c_in = x.shape
    c_out = packed.shape[0]
    dw, ds, dx = (hip.DeviceArray.from_numpy(a) for a in (packed, scales, x))
    out = hip.DeviceArray((batch, c_out), np.float32)
    pkv.q4_matmul(dw, ds, dx, out, c_in, c_out, batch)
    return out.numpy()


def test_reference_patterns(gpu):
    # test_q4_4row_tiling.mojo:119-136: c_in 2816, 67 rows (a partial row tile), one vector.
    print("[q4] reference patterns", flush=True)
    c_in, c_out = 2816, 67
    x = ((np.arange(c_in) % 31 - 15).astype(np.float32) * np.float32(0.02)).astype(np.float32)
    packed = ((np.arange(c_out * (c_in // 2), dtype=np.int64) * 13 + 7) & 255).astype(np.uint8)
    packed = packed.reshape(c_out, -1)
    scales = ((((np.arange(c_out * (c_in // 32)) % 19) + 1).astype(np.float32) * np.float32(0.002))
              .astype(np.float32).reshape(c_out, -1))
    got = _run(packed, scales, x.reshape(1, -1))[0]
    ref = O.q4_matmul_vec(packed, scales, x)
    assert np.max(np.abs(got - ref)) <= 1e-4


@pytest.mark.parametrize("c_in,c_out,batch", [
    (4096, 2816, 32),  # sliding layers' Wo at the decode batch
    (8192, 2816, 32),  # global layers' Wo (16 q heads x 512)
    (4096, 2816, 5),   # a verify-sized batch
    (8192, 1000, 64),  # the largest batch, partial row tile
    (96, 17, 3),       # a single workgroup per row group
    (2848, 300, 40),   # three column tiles, 89 blocks: row groups split over workgroups
    (4128, 129, 17),   # two column tiles, a 129-row matrix (one row in the last group)
    (32, 5, 1),        # one block, one sequence
], ids=["wo-sliding", "wo-global", "b5", "b64", "small", "b40-odd", "b17-odd", "tiny"])
def test_wo_shapes_within_dot_bound(gpu, c_in, c_out, batch):
    print(f"[q4] c_in={c_in} c_out={c_out} batch={batch}", flush=True)
    rng = np.random.default_rng(c_in + c_out + batch)
    packed, scales = O.quantize_q4_0((rng.standard_normal((c_out, c_in)) * 0.05).astype(np.float32))
    x = rng.standard_normal((batch, c_in)).astype(np.float32)
    got = _run(packed, scales, x)
    w = _dequant(packed, scales)
    absum = np.abs(x.astype(np.float64)) @ np.abs(w).T  # [batch][c_out]
    for s in range(batch):
        exact = O.q4_matmul_f64(packed, scales, x[s])
        ref = O.q4_matmul_vec(packed, scales, x[s])
        bound = 1e-6 * absum[s]
        assert np.all(np.abs(ref - exact) <= bound), "the fp32 oracle itself exceeds the bound"
        err = np.abs(got[s].astype(np.float64) - exact)
        assert np.all(err <= bound), f"sequence {s}: max err / bound {np.max(err / bound)}"



def test_workspace_reused_across_calls_and_shapes(gpu):
    """One zero-filled workspace serves a sequence of calls of different shapes (the row
    groups' arrival counts return to zero after each call): every output equals the one a
    fresh workspace gives, bit for bit."""
    print("[q4] workspace reuse", flush=True)
    rng = np.random.default_rng(7)
    shapes = [(8192, 2816, 32), (4096, 2816, 32), (2848, 300, 40), (8192, 2816, 32), (96, 17, 3)]
    need = max(pkv.lib.load().pkv_q4_matmul_workspace_size(ci, co, b) for ci, co, b in shapes)
    ws = hip.DeviceArray((need,), np.uint8, zero=True)
    for c_in, c_out, batch in shapes:
        packed = rng.integers(0, 256, (c_out, c_in // 2), dtype=np.uint8)
        scales = (rng.random((c_out, c_in // 32)) * 0.01 + 0.001).astype(np.float32)
        x = rng.standard_normal((batch, c_in)).astype(np.float32)
        dw, ds, dx = (hip.DeviceArray.from_numpy(a) for a in (packed, scales, x))
        reused = hip.DeviceArray((batch, c_out), np.float32)
        pkv.q4_matmul(dw, ds, dx, reused, c_in, c_out, batch, workspace=ws)
        fresh = _run(packed, scales, x)
        assert np.array_equal(reused.numpy(), fresh), f"shape {(c_in, c_out, batch)}"
