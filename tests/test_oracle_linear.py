"""Pins the oracle's linear layer (the reference's GEMM test reference, tests/test_cuda.cpp:27-47, with the
epilogues of src/backend/cuda/kernels.cuh:25-30) against numpy's float64 matmul, the identity weight and silu's
closed form."""
import numpy as np
import pytest

import oracle


def _f16(rng, shape, scale):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


@pytest.mark.parametrize("M,N,K", [(1, 16, 32), (3, 130, 64), (13, 200, 96), (64, 48, 128)])
def test_linear_matches_float64_matmul(M, N, K):
    rng = np.random.default_rng(M * 1000 + N)
    a, w = _f16(rng, (M, K), 1.0), _f16(rng, (N, K), 0.05)
    want = a.astype(np.float64) @ w.astype(np.float64).T
    got = oracle.linear(a, w, 0)
    assert np.allclose(got, want.astype(np.float32), rtol=0, atol=np.abs(want).max() * 2 ** -23 * 4)
    np.testing.assert_array_equal(oracle.linear(a, w, 1), got)
    c = rng.standard_normal((M, N)).astype(np.float32)
    np.testing.assert_array_equal(oracle.linear(a, w, 2, c), c + got)


def test_identity_weight_returns_the_input():
    rng = np.random.default_rng(7)
    a = _f16(rng, (5, 64), 3.0)
    got = oracle.linear(a, np.eye(64, dtype=np.float16), 0)
    np.testing.assert_array_equal(got, a.astype(np.float32))


def test_silu_mul_closed_form():
    """Interleaved gate/up rows: with W = [e_0; e_1; e_2; e_3] the gates are a[:, 0], a[:, 2] and the ups
    a[:, 1], a[:, 3], so out[m, j] = silu(a[m, 2j]) * a[m, 2j + 1]."""
    rng = np.random.default_rng(11)
    a = _f16(rng, (4, 32), 2.0)
    w = np.eye(32, dtype=np.float16)[:4]
    got = oracle.linear(a, w, 3)
    g, u = a[:, 0::2][:, :2].astype(np.float64), a[:, 1::2][:, :2].astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=1e-7)


@pytest.mark.parametrize("epilogue", [0, 1, 2, 3])
def test_threaded_linear_is_bit_identical(epilogue):
    """The threaded form spreads the same double sums over threads: every epilogue, bit for bit."""
    rng = np.random.default_rng(12)
    a, w = _f16(rng, (37, 96), 1.0), _f16(rng, (64, 96), 0.1)
    c = rng.standard_normal((37, 32 if epilogue == 3 else 64)).astype(np.float32)
    one = oracle.linear(a, w, epilogue, c if epilogue == 2 else None)
    many = oracle.linear(a, w, epilogue, c if epilogue == 2 else None, threads=7)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))
