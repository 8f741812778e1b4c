"""The GPU sampler (ember_hip_sample / ember_hip_token_probs) against the oracle's host sampler, as the reference
checks its CUDA sampler (tests/test_cuda.cpp:137-186): greedy and top-k 1 take the argmax; 2000 draws with
temperature 0.8, top-k 40, top-p 0.9 stay inside the host's kept set and follow its distribution; and the same
(seed, counter) gives the same token as the host sampler, draw for draw. Token probabilities equal the host
distribution's within 1e-4 relative."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from ember_amd import _lib

pytestmark = pytest.mark.gpu


def _params(rows):
    p = (_lib.SampleParams * len(rows))()
    for i, (t, top_p, top_k, min_p, seed, counter) in enumerate(rows):
        p[i].temperature, p[i].top_p, p[i].top_k, p[i].min_p, p[i].seed, p[i].counter = t, top_p, top_k, min_p, seed, counter
    return torch.frombuffer(bytearray(p), dtype=torch.uint8).cuda()


def gpu_sample(logits: np.ndarray, rows) -> list:
    x = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).cuda()
    R, V = x.shape
    params = _params(rows)
    out = torch.full((R,), -1, dtype=torch.int32, device="cuda")
    a = _lib.SampleArgs()
    a.logits, a.R, a.vocab, a.params, a.out = x.data_ptr(), R, V, params.data_ptr(), out.data_ptr()
    _lib.check(_lib.lib().ember_hip_sample(ctypes.byref(a), torch.cuda.current_stream().cuda_stream), "sample")
    torch.cuda.synchronize()
    return out.cpu().tolist()


def gpu_probs(logits: np.ndarray, rows, queries) -> np.ndarray:
    x = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).cuda()
    R, V = x.shape
    params = _params(rows)
    q = torch.tensor(queries, dtype=torch.int32).reshape(-1, 2)
    r_dev, t_dev = q[:, 0].contiguous().cuda(), q[:, 1].contiguous().cuda()
    out = torch.full((q.shape[0],), -1.0, device="cuda")
    a = _lib.ProbArgs()
    a.logits, a.vocab, a.params, a.rows, a.tokens = x.data_ptr(), V, params.data_ptr(), r_dev.data_ptr(), t_dev.data_ptr()
    a.n, a.out, a.R = q.shape[0], out.data_ptr(), R
    _lib.check(_lib.lib().ember_hip_token_probs(ctypes.byref(a), torch.cuda.current_stream().cuda_stream), "probs")
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.fixture(scope="module")
def logits():
    return np.random.default_rng(7).normal(0.0, 3.0, 5000).astype(np.float32)


def test_greedy_and_top_k_one(logits):
    best = int(np.argmax(logits))
    got = gpu_sample(np.stack([logits, logits]), [(0.0, 1.0, 0, 0.0, 0, 0), (1.0, 1.0, 1, 0.0, 5, 3)])
    assert got == [best, best]
    tied = logits.copy()
    tied[[3, 4000]] = tied.max() + 1.0  # ties go to the lower id
    assert gpu_sample(tied[None, :], [(0.0, 1.0, 0, 0.0, 0, 0)]) == [3]


@pytest.mark.parametrize("t,top_p,top_k,min_p", [(0.8, 0.9, 40, 0.0), (1.0, 0.95, 0, 0.0), (1.2, 1.0, 0, 0.02),
                                                 (0.7, 0.8, 100, 0.01)])
def test_draws_follow_the_host_sampler(logits, t, top_p, top_k, min_p):
    R = 2000
    rows = [(t, top_p, top_k, min_p, 99, c) for c in range(R)]
    toks = np.array(gpu_sample(np.tile(logits, (R, 1)), rows))
    kept, probs = oracle.sampling_distribution(logits, t, top_p, top_k, min_p)
    assert set(toks.tolist()) <= set(kept.tolist()), "a draw outside the host's kept set"
    f0 = float((toks == kept[0]).mean())
    assert abs(f0 - probs[0]) < 4 * np.sqrt(probs[0] * (1 - probs[0]) / R) + 0.01
    host = [oracle.sample(logits, t, top_p, top_k, min_p, seed=99, counter=c) for c in range(200)]
    assert toks[:200].tolist() == host, "the GPU and host samplers draw different tokens for the same noise"


def test_token_probs_match_the_host_distribution(logits):
    kept, probs = oracle.sampling_distribution(logits, 0.8, 0.9, 40, 0.0)
    outside = int(np.argsort(logits)[0])
    rows = [(0.8, 0.9, 40, 0.0, 1, 2), (0.0, 1.0, 0, 0.0, 0, 0)]
    q = [(0, int(kept[0])), (0, int(kept[-1])), (0, int(kept[len(kept) // 2])), (0, outside),
         (1, int(np.argmax(logits))), (1, outside), (2, 5), (0, 5000)]  # the last two: a row and a token out of range
    got = gpu_probs(np.stack([logits, logits]), rows, q)
    np.testing.assert_allclose(got[:3], probs[[0, -1, len(kept) // 2]], rtol=1e-4)
    assert got[3] == 0.0 and got[4] == 1.0 and got[5] == 0.0 and got[6] == 0.0 and got[7] == 0.0


@pytest.mark.parametrize("V", [4999, 5000])
def test_rows_of_any_length_and_ties_across_threads(logits, V):
    """Rows of 4999 and 5000 logits: the draws are the host sampler's, and greedy takes the first largest of a tie
    whose tokens lie in different threads' elements."""
    x = logits[:V].copy()
    x[[6, 9, 4000]] = x.max() + 1.0
    host = [oracle.sample(x, 0.8, 0.9, 40, 0.0, seed=5, counter=c) for c in range(64)]
    rows = [(0.8, 0.9, 40, 0.0, 5, c) for c in range(64)] + [(0.0, 1.0, 0, 0.0, 0, 0)]
    got = gpu_sample(np.tile(x, (65, 1)), rows)
    assert got[:64] == host
    assert got[64] == 6


def test_full_vocabulary_rows_and_batch_invariance():
    """Qwen3's 151,936-token vocabulary: each row's token does not depend on the other rows of the launch."""
    rng = np.random.default_rng(11)
    x = rng.normal(0.0, 2.0, (6, 151936)).astype(np.float32)
    rows = [(0.9, 0.9, 0, 0.0, 7, c) for c in range(6)]
    together = gpu_sample(x, rows)
    alone = [gpu_sample(x[i:i + 1], rows[i:i + 1])[0] for i in range(6)]
    assert together == alone
    assert together == [oracle.sample(x[i], 0.9, 0.9, 0, 0.0, seed=7, counter=i) for i in range(6)]


def _tied_rows():
    """Rows whose top-k or top-p cut falls inside a run of exactly equal logits (sampling_host.cpp:31-58 keeps the
    lower ids first)."""
    rng = np.random.default_rng(23)
    base = rng.normal(0.0, 1.0, 3000).astype(np.float32)
    k_tie = base.copy()
    k_tie[np.argsort(base)[-5:]] += 8.0                  # 5 clear leaders
    ties_k = np.array([17, 400, 401, 1999, 2500, 2999])
    k_tie[ties_k] = np.float32(6.5)                      # 6 tokens tied just below them; top-k 8 keeps 3 of them
    p_tie = np.full(3000, -10.0, np.float32)
    ties_p = np.array([5, 77, 78, 900, 1500, 2100, 2200, 2901])
    p_tie[ties_p] = np.float32(4.0)                      # 8 equal leaders: top-p 0.3 keeps the 3 lowest ids
    return [(k_tie, (1.0, 1.0, 8, 0.0), ties_k), (p_tie, (1.0, 0.3, 0, 0.0), ties_p),
            (p_tie, (0.9, 0.55, 6, 0.0), ties_p), (k_tie, (1.3, 0.999, 7, 0.0), ties_k)]


@pytest.mark.parametrize("case", range(4))
def test_ties_at_the_top_k_and_top_p_cuts(case):
    """Tokens tied at a top-k or top-p boundary: the GPU keeps the same tokens as the host sampler (the lowest ids of
    the tie, as many as the count or mass asks for), gives the same probabilities, and draws the same tokens."""
    x, (t, top_p, top_k, min_p), ties = _tied_rows()[case]
    kept, probs = oracle.sampling_distribution(x, t, top_p, top_k, min_p)
    in_tie = np.intersect1d(kept, ties)
    assert 0 < in_tie.size < ties.size, "the case must cut inside the tie"
    assert np.array_equal(in_tie, np.sort(ties)[:in_tie.size]), "the host keeps the lowest ids of a tie"
    rows = [(t, top_p, top_k, min_p, 31, 0)]
    q = [(0, int(i)) for i in ties] + [(0, int(kept[0]))]
    got = gpu_probs(x[None, :], rows, q)
    want = np.array([probs[list(kept).index(i)] if i in kept else 0.0 for i in ties] + [probs[0]], np.float32)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=0.0)
    R = 400
    toks = gpu_sample(np.tile(x, (R, 1)), [(t, top_p, top_k, min_p, 31, c) for c in range(R)])
    assert set(toks) <= set(kept.tolist()), "a draw outside the host's kept set"
    assert toks[:100] == [oracle.sample(x, t, top_p, top_k, min_p, seed=31, counter=c) for c in range(100)]
