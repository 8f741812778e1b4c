"""The oracle's sampler and dot product against the reference's own code, compiled from the reference tree into
oracle/_ref by oracle/Makefile (`make ref`): src/backend/sampling_host.cpp:10-87 with sampling_rng.hpp:22-33, and
src/backend/cpu/cpu_kernels_avx2.cpp:27-69. Every value is compared bit for bit: the Gumbel composition (the
mixing constant, the 24-bit uniform, the double log), the kept sets and probabilities of every filter (with tied
logits at the top-k and top-p cuts), the draws, and the AVX2 dot product's lane order. Skipped where oracle/_ref
was not built (no reference tree)."""
import numpy as np
import pytest

import oracle

REF = oracle.ref_lib()
pytestmark = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (no reference tree here)")

_F32P = oracle._F32P
_I32P = oracle._I32P


def _ref_distribution(x, temperature, top_p, top_k, min_p):
    x = np.ascontiguousarray(x, np.float32)
    toks = np.empty(x.size, np.int32)
    probs = np.empty(x.size, np.float32)
    n = REF.ember_ref_sampling_distribution(oracle._p(x, _F32P), x.size, temperature, top_p, top_k, min_p,
                                            oracle._p(toks, _I32P), oracle._p(probs, _F32P))
    return toks[:n].copy(), probs[:n].copy()


def _ref_sample(x, temperature, top_p, top_k, min_p, seed, counter):
    x = np.ascontiguousarray(x, np.float32)
    return int(REF.ember_ref_sample_host(oracle._p(x, _F32P), x.size, temperature, top_p, top_k, min_p, seed, counter))


def test_rng_mix_matches_reference():
    rng = np.random.default_rng(1)
    for z in rng.integers(0, 2 ** 63, 2000, dtype=np.uint64).tolist() + [0, 2 ** 64 - 1, 0x9E3779B97F4A7C15]:
        assert oracle.rng_mix(z) == REF.ember_ref_rng_mix(z)


def test_gumbel_noise_matches_reference_bit_for_bit():
    rng = np.random.default_rng(2)
    seeds = rng.integers(0, 2 ** 63, 40, dtype=np.uint64).tolist() + [0, 1, 99, 2 ** 64 - 1]
    for seed in seeds:
        for counter in [0, 1, 7, 12345, 2 ** 40 + 3]:
            ids = rng.integers(0, 151936, 64).tolist() + [0, 1, 151935]
            got = np.array([oracle.gumbel(seed, counter, t) for t in ids], np.float32)
            want = np.array([REF.ember_ref_gumbel_noise(seed, counter, t) for t in ids], np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seed, counter)


def _logits(rng, vocab, kind):
    if kind == "normal":
        return (rng.standard_normal(vocab) * 3).astype(np.float32)
    if kind == "ties":  # few distinct values: ties at every cut
        return rng.integers(-4, 5, vocab).astype(np.float32)
    x = np.full(vocab, -2.0, np.float32)  # one clear winner, then a tied plateau
    x[rng.integers(0, vocab)] = 5.0
    return x


CASES = [(t, p, k, m) for t in (1e-6, 0.5, 1.0, 1.7) for p in (1.0, 0.9, 0.5) for k in (0, 1, 5, 50)
         for m in (0.0, 0.05)]


@pytest.mark.parametrize("vocab,kind", [(1, "normal"), (2, "ties"), (17, "ties"), (300, "normal"), (300, "ties"),
                                        (1000, "plateau"), (4096, "normal")])
def test_sampling_distribution_matches_reference(vocab, kind):
    rng = np.random.default_rng(vocab * 7 + len(kind))
    x = _logits(rng, vocab, kind)
    for t, p, k, m in CASES:
        got_t, got_p = oracle.sampling_distribution(x, temperature=t, top_p=p, top_k=k, min_p=m)
        want_t, want_p = _ref_distribution(x, t, p, k, m)
        assert np.array_equal(got_t, want_t), (t, p, k, m)
        assert np.array_equal(got_p.view(np.uint32), want_p.view(np.uint32)), (t, p, k, m)


@pytest.mark.parametrize("vocab,kind", [(17, "ties"), (300, "normal"), (1000, "plateau"), (4096, "ties")])
def test_draws_match_reference(vocab, kind):
    rng = np.random.default_rng(vocab + 3)
    x = _logits(rng, vocab, kind)
    for t, p, k, m in CASES[::3]:
        for seed in (0, 5, 2 ** 63 + 11):
            for counter in range(0, 40, 3):
                got = oracle.sample(x, temperature=t, top_p=p, top_k=k, min_p=m, seed=seed, counter=counter)
                assert got == _ref_sample(x, t, p, k, m, seed, counter), (t, p, k, m, seed, counter)


def test_dot_matches_reference_avx2():
    """Lengths that are multiples of 8, where the reference's dot product is its intrinsics alone: 16-wide FMA
    steps on two accumulators, one 8-wide step, then the horizontal sum in its lane order. (Its scalar tail for
    other lengths rounds as the compiler contracts and vectorizes it: the reference's own GCC -O3 -mfma build
    multiplies groups of four unfused and fuses the last one to three. The path never takes the tail: head_dim
    128, hidden sizes multiples of 32.)"""
    flags = open("/proc/cpuinfo").read().split()
    if "avx2" not in flags or "fma" not in flags:
        pytest.skip("no AVX2 + FMA on this CPU: the oracle takes its scalar dot product")
    rng = np.random.default_rng(4)
    for n in list(range(0, 129, 8)) + [1000, 1024, 2048, 4096, 4104]:
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        got = np.float32(oracle.dot(a, b))
        ap, bp = np.ascontiguousarray(a), np.ascontiguousarray(b)
        want = np.float32(REF.ember_ref_dot_avx2(oracle._p(ap, _F32P), oracle._p(bp, _F32P), n))
        assert got.view(np.uint32) == want.view(np.uint32), n
