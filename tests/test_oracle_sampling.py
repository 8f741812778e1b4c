"""Pins the oracle's sampler (src/backend/sampling_host.cpp:20-87, src/backend/sampling_rng.hpp:22-33):
SplitMix64's published outputs, the Gumbel(0, 1) moments, each filter against a numpy restatement of its own,
and the Gumbel-max draw's frequencies against the distribution."""
import numpy as np
import pytest

import oracle

GOLDEN = 0x9E3779B97F4A7C15
MASK = 0xFFFFFFFFFFFFFFFF


def test_rng_mix_is_splitmix64():
    # SplitMix64 from state 0: the k-th output is the mix of state k * golden (published test vectors)
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC, 0x1B39896A51A8749B]
    assert [oracle.rng_mix((k * GOLDEN) & MASK) for k in range(5)] == want


def test_gumbel_noise_moments():
    g = np.array([oracle.gumbel(seed, counter, tok) for seed in (1, 99) for counter in range(200) for tok in range(250)])
    assert abs(g.mean() - 0.5772156649) < 0.01          # Euler-Mascheroni
    assert abs(g.var() - np.pi ** 2 / 6) < 0.04
    assert oracle.gumbel(5, 6, 7) == oracle.gumbel(5, 6, 7) and oracle.gumbel(5, 6, 7) != oracle.gumbel(5, 6, 8)


def _numpy_distribution(x, t, top_p, top_k, min_p):
    v = x.astype(np.float64) / t
    order = np.lexsort((np.arange(v.size), -v))  # descending value, ties to the lower id
    if 0 < top_k < v.size:
        order = order[:top_k]
    p = np.exp(v[order] - v[order[0]])
    p /= p.sum()
    n = p.size
    if top_p < 1.0:
        n = int(np.searchsorted(np.cumsum(p), top_p) + 1)
    if min_p > 0.0:
        keep = p[:n] >= min_p * p[0]
        n = int(keep.argmin()) if not keep.all() else n
        n = max(n, 1)
    return order[:n], p[:n] / p[:n].sum()


@pytest.mark.parametrize("t,top_p,top_k,min_p", [
    (1.0, 1.0, 0, 0.0), (0.8, 0.9, 40, 0.0), (1.3, 0.5, 0, 0.0), (0.7, 1.0, 10, 0.0), (1.0, 1.0, 0, 0.05),
    (0.9, 0.95, 100, 0.02)])
def test_sampling_distribution_matches_numpy(rng, t, top_p, top_k, min_p):
    x = rng.normal(0, 3, 5000).astype(np.float32)
    toks, probs = oracle.sampling_distribution(x, t, top_p, top_k, min_p)
    wt, wp = _numpy_distribution(x, t, top_p, top_k, min_p)
    assert np.array_equal(toks, wt)
    np.testing.assert_allclose(probs, wp, rtol=1e-5, atol=1e-9)
    assert abs(probs.sum() - 1.0) < 1e-5


def test_greedy_and_top_k_one_take_the_argmax(rng):
    x = rng.normal(0, 3, 1000).astype(np.float32)
    x[17] = x[611] = x.max() + 1.0  # a tie: the lower id wins
    for params in ({"temperature": 0.0}, {"temperature": 1.0, "top_k": 1}):
        toks, probs = oracle.sampling_distribution(x, **params)
        assert toks.tolist() == [17] and probs.tolist() == [1.0]
        assert all(oracle.sample(x, seed=3, counter=c, **params) == 17 for c in range(5))


def test_draw_frequencies_follow_the_distribution():
    x = np.array([2.0, 1.5, 1.0, 0.2, -1.0, -3.0, 0.9, 1.4], np.float32)
    toks, probs = oracle.sampling_distribution(x, 0.8, 0.9, 6, 0.0)
    R = 20000
    draws = np.array([oracle.sample(x, 0.8, 0.9, 6, 0.0, seed=99, counter=c) for c in range(R)])
    assert set(draws.tolist()) <= set(toks.tolist())      # never outside the kept set
    for tok, p in zip(toks, probs):
        f = (draws == tok).mean()
        assert abs(f - p) < 4 * np.sqrt(p * (1 - p) / R) + 1e-3, (tok, f, p)
