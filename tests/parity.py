"""The attention-output parity rule used by every GPU test and by smoke().

Tolerances (north star; metric max |x - ref| / (|ref| + 1e-3), test_attention.mojo:259-266):
  fp32 pools: 1e-4 against the reference's fp32 CPU path (the oracle's restatement of
              attention.mojo:151-294).
  bf16 pools: 2e-2 against that path run on the same bf16-rounded values.

The reference's fp32 path is itself an approximation of exact attention: its own
float64 test oracle (test_attention.mojo:123-163) bounds it at 1e-4, and on some inputs
(head_dim 512 dots, unscaled large scores) its rounding error alone exceeds 1e-4. The
fp32 GPU path accumulates in double, so for fp32 pools it must also sit within 1e-5 of
the float64 attention; when the fp32 reference is farther than 1e-4 from exact, the
GPU is held to the exact result plus the reference's own distance from it.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

TOL_F32 = 1e-4
TOL_BF16 = 2e-2
TOL_EXACT = 1e-5  # fp32-pool GPU output vs the float64 attention


def check(gpu, ref32, ref64=None, bf16=False, what=""):
    """Asserts the parity rule; returns (err_vs_ref32, err_vs_f64 or None)."""
    gpu = np.asarray(gpu)
    assert np.all(np.isfinite(gpu)), f"{what}: non-finite output"
    e32 = O.max_rel_err(gpu, ref32)
    if bf16:
        assert e32 <= TOL_BF16, f"{what}: bf16 err {e32} > {TOL_BF16}"
        return e32, None
    if ref64 is None:
        assert e32 <= TOL_F32, f"{what}: err {e32} > {TOL_F32}"
        return e32, None
    e64 = O.max_rel_err(gpu, ref64)
    assert e64 <= TOL_EXACT, f"{what}: err vs float64 {e64} > {TOL_EXACT}"
    ref_own = O.max_rel_err(ref32, ref64)
    assert e32 <= max(TOL_F32, ref_own + TOL_EXACT), \
        f"{what}: err {e32} vs fp32 reference (reference's own error {ref_own})"
    return e32, e64
