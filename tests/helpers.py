"""Test helpers: random paged steps, and an independent float64 attention reference.

The float64 reference gathers each sequence's keys and values into dense
arrays with numpy fancy indexing (its own route from (sequence, position) to
memory, not the oracle's cache_offset) and evaluates the textbook
softmax(q K^T / sqrt(D)) V.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

PAGE = 16
D = 128


@dataclass
class Step:
    positions: np.ndarray    # [T]
    query_start: np.ndarray  # [S+1]
    tables: np.ndarray       # [S, max_blocks]
    token_seq: np.ndarray    # [T]

    @property
    def T(self):
        return int(self.positions.size)

    @property
    def S(self):
        return int(self.tables.shape[0])


def make_step(rng, ctx_after, new_tokens, num_blocks, max_blocks=None) -> Step:
    """Sequences whose context is ctx_after[s] after appending new_tokens[s] tokens; pages scattered by a
    seeded permutation of the pool (disjoint between sequences)."""
    ctx_after = np.asarray(ctx_after, int)
    new_tokens = np.asarray(new_tokens, int)
    pages = (ctx_after + PAGE - 1) // PAGE
    mb = int(max_blocks or max(1, pages.max()))
    assert pages.sum() <= num_blocks, "pool too small"
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.zeros((len(ctx_after), mb), np.int32)
    at = 0
    for s, p in enumerate(pages):
        tables[s, :p] = perm[at:at + p]
        at += p
    positions, token_seq, qs = [], [], [0]
    for s, (c, n) in enumerate(zip(ctx_after, new_tokens)):
        positions += list(range(c - n, c))
        token_seq += [s] * n
        qs.append(qs[-1] + n)
    return Step(np.array(positions, np.int32), np.array(qs, np.int32), tables, np.array(token_seq, np.int32))


def dense_kv(cache, tables_row, ctx):
    """[ctx, n_kv, D] keys (or values) of one sequence, gathered page by page. cache: [NB, n_kv, 16, D]."""
    pages = cache[tables_row[: (ctx + PAGE - 1) // PAGE]]          # [p, n_kv, 16, D]
    return pages.transpose(0, 2, 1, 3).reshape(-1, cache.shape[1], cache.shape[3])[:ctx]


def attention_f64(q, step: Step, k_cache, v_cache, n_heads, n_kv):
    """Textbook causal GQA attention in float64. q [T, H, D]; caches [NB, n_kv, 16, D] float."""
    G = n_heads // n_kv
    out = np.zeros(q.shape, np.float64)
    for t in range(step.T):
        s, ctx = step.token_seq[t], step.positions[t] + 1
        K = dense_kv(k_cache, step.tables[s], ctx).astype(np.float64)
        V = dense_kv(v_cache, step.tables[s], ctx).astype(np.float64)
        for h in range(n_heads):
            sc = K[:, h // G, :] @ q[t, h].astype(np.float64) / np.sqrt(q.shape[-1])
            w = np.exp(sc - sc.max())
            out[t, h] = (w / w.sum()) @ V[:, h // G, :]
    return out


def rel_err(got, want):
    """max |got - want| / max |want| per (token, head) vector, worst over vectors."""
    g = np.asarray(got, np.float64).reshape(-1, np.shape(got)[-1])
    w = np.asarray(want, np.float64).reshape(-1, np.shape(want)[-1])
    den = np.maximum(np.abs(w).max(axis=1), 1e-30)
    return float((np.abs(g - w).max(axis=1) / den).max())
