"""Pins the oracle's f16 <-> f32 conversions (src/common/fp16.hpp:25-71) to numpy's IEEE float16."""
import numpy as np

import oracle


def test_f16_to_f32_exhaustive():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # signed zeros included


def test_f32_to_f16_round_to_nearest_even(rng):
    edge = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, np.inf, -np.inf,
                     6.1035156e-05, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.98023259e-08, 1e-8, 1e-30,
                     0.1, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2049.0, 2051.0], np.float32)
    rand = np.concatenate([
        rng.standard_normal(200000).astype(np.float32),
        (rng.standard_normal(200000) * 1e-5).astype(np.float32),    # subnormal range of f16
        (rng.standard_normal(200000) * 3e4).astype(np.float32),     # near overflow
        rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32),  # every bit pattern class
    ])
    x = np.concatenate([edge, rand])
    got = oracle.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all((got[nan] & 0x3ff) != 0)  # NaN stays NaN


def test_round_trip_of_every_half():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = ~np.isnan(bits.view(np.float16))
    back = oracle.f32_to_f16(oracle.f16_to_f32(bits))
    assert np.array_equal(back[finite], bits[finite])
