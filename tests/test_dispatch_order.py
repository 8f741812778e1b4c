"""The decode work list's launch order (ember_kv_dispatch_order, host only). Its contract: every item exactly once,
-1 only for empty items inside the first round, the plain largest-first order when the column model does not apply,
and, under a model of the dispatcher (work-group b on the CU of b mod n_cu while every CU has a free slot, later ones
on the earliest-freed slot of their XCD, each CU running its work-groups in launch order at one page per unit of time),
a heaviest CU no heavier than the largest-first order gives. The reference launches a dense (token, kv head, split)
grid (k_attention.cu:372-386) and has no counterpart: these checks pin the intent, the GPU tests pin the results."""
import heapq

import numpy as np
import pytest

from ember_amd.paged_kv import dispatch_order

N_CU, XCDS, SLOTS, KVH, SPLIT = 256, 8, 4, 8, 512


def _items(rng, n_seqs, lo, hi):
    """Page counts of the decode items of n_seqs sequences with contexts U[lo, hi] in 512-key splits."""
    pages = []
    for ctx in rng.integers(lo, hi + 1, n_seqs):
        for s in range(0, int(ctx), SPLIT):
            pages.append((min(SPLIT, int(ctx) - s) + 15) // 16)
    return pages


def _simulate(order, pages, n_kv=KVH, n_cu=N_CU, slots=SLOTS):
    """Per-CU page totals under the dispatcher model above (item -1: a work-group that exits at once)."""
    wgs = [(i, k) for i in order for k in range(n_kv)]
    load = np.zeros(n_cu)
    free = [[] for _ in range(XCDS)]  # per XCD: heap of (time a slot frees, cu)
    busy_until = np.zeros(n_cu)
    for b, (item, _) in enumerate(wgs):
        cost = 0 if item < 0 else pages[item]
        if b < n_cu * slots:
            cu = b % n_cu
        else:
            _, cu = heapq.heappop(free[b % XCDS])
        busy_until[cu] += cost  # the CU runs its work-groups one after another, in launch order
        load[cu] += cost
        heapq.heappush(free[cu % XCDS], (busy_until[cu], cu))
    return load


def test_every_item_once_and_fallbacks():
    rng = np.random.default_rng(5)
    pages = _items(rng, 32, 256, 4096)
    order = dispatch_order(pages, KVH, N_CU, SLOTS)
    assert sorted(i for i in order if i >= 0) == list(range(len(pages)))
    first_round = N_CU // KVH * SLOTS
    assert all(i >= 0 for i in order[first_round:]), "empty items only inside the first round"
    largest_first = sorted(range(len(pages)), key=lambda i: -pages[i])  # Python's sort is stable, as the C++ is
    assert dispatch_order(pages, KVH, N_CU, 0) == largest_first  # occupancy unknown
    assert dispatch_order(pages, 3, N_CU, SLOTS) == largest_first  # kv heads that do not divide the CUs
    many = _items(rng, 64, 2048, 4096)  # more than two rounds: the dispatcher balances by itself
    assert len(many) > 2 * first_round
    assert dispatch_order(many, KVH, N_CU, SLOTS) == sorted(range(len(many)), key=lambda i: -many[i])
    assert dispatch_order([], KVH, N_CU, SLOTS) == []


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5, 6, 7])
def test_config2_like_lists_put_the_overflow_on_light_cus(seed):
    """BASELINE config 2's shape: 32 sequences, contexts U[256, 4096], 8 kv heads: about 140 items, just over one
    round of 128 item positions. Largest first lets the overflow land on CUs that already hold four full splits."""
    rng = np.random.default_rng(seed)
    pages = _items(rng, 32, 256, 4096)
    cols = N_CU // KVH
    assert cols * SLOTS < len(pages) <= 2 * cols * SLOTS
    order = dispatch_order(pages, KVH, N_CU, SLOTS)
    # first round: each column's items smallest first
    for c in range(cols):
        col = [order[q] for q in range(c, cols * SLOTS, cols) if order[q] >= 0]
        assert [pages[i] for i in col] == sorted(pages[i] for i in col)
    new = _simulate(order, pages).max()
    old = _simulate(sorted(range(len(pages)), key=lambda i: -pages[i]), pages).max()
    lower = max(max(pages), -(-sum(pages) * KVH // N_CU))  # no schedule beats the mean or the largest item
    assert lower <= new <= old, (new, old)
    assert new <= lower + max(pages), (new, lower)  # the greedy packing's bound: the mean plus one item


def test_one_round_packs_columns_without_overflow():
    rng = np.random.default_rng(9)
    pages = _items(rng, 20, 256, 4096)
    cols = N_CU // KVH
    assert len(pages) <= cols * SLOTS
    order = dispatch_order(pages, KVH, N_CU, SLOTS)
    assert len(order) <= cols * SLOTS
    loads = [sum(pages[order[q]] for q in range(c, len(order), cols) if order[q] >= 0) for c in range(cols)]
    # largest-first greedy packing: no column exceeds the mean by more than its smallest item
    assert max(loads) <= sum(pages) / cols + max(pages)
