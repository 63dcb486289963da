"""The FP8 group scale max(amax, 1e-10) / 448 without a division.

The kernels form it as (x / 7) * 2^-6, with x / 7 as q0 = x * RN(1/7)
corrected by one fused multiply-add of the remainder, q = fma(fma(-q0, 7,
x), RN(1/7), q0). For every fp32 significand (x in [1, 2); the exponent only
scales the operands and results exactly, all of them normal for x >= 1e-10)
that must be the correctly rounded quotient, and so (x / 7) * 2^-6 equals
the reference's x / 448 (attention.py:780-781) bit for bit. Checked here
exhaustively, with each fp32 fma evaluated exactly in float64 and rounded
once: the products x * RN(1/7), q0 * 7 and r * RN(1/7) have at most 48
significant bits, and the sums they enter are exact in float64 (the
remainder r = x - 7 q0 is an fp32 value, and r * RN(1/7) is below 2^-23 of
q0).
"""

import numpy as np


def test_seventh_by_one_fma_correction_is_correctly_rounded_for_every_significand():
    x = (np.arange(1 << 23, dtype=np.uint32) | np.uint32(0x3F800000)).view(np.float32)
    c = np.float32(1.0) / np.float32(7.0)
    q0 = x * c                                                  # fp32 multiply, RN
    r = (x.astype(np.float64) - q0.astype(np.float64) * 7.0).astype(np.float32)
    assert np.array_equal(r.astype(np.float64), x.astype(np.float64) - q0.astype(np.float64) * 7.0)
    q = (r.astype(np.float64) * np.float64(c) + q0.astype(np.float64)).astype(np.float32)
    want = x / np.float32(7.0)                                  # IEEE division, RN
    assert np.array_equal(q.view(np.uint32), want.view(np.uint32))
    # and the scale itself over a spread of magnitudes, including the floor
    amax = np.concatenate([np.float32([0.0, 1e-10, 1e-12, 448.0, 3.0e38]),
                           np.random.default_rng(0).lognormal(0, 6, 100000).astype(np.float32)])
    xs = np.maximum(amax, np.float32(1e-10))
    q0 = xs * c
    r = (xs.astype(np.float64) - q0.astype(np.float64) * 7.0).astype(np.float32)
    q = (r.astype(np.float64) * np.float64(c) + q0.astype(np.float64)).astype(np.float32)
    assert np.array_equal((q * np.float32(0.015625)).view(np.uint32),
                          (xs / np.float32(448.0)).view(np.uint32))
