"""Page placement: the product BlockManager (C++ through the C ABI) and the
oracle's restatement of src/kvcache/block_manager.cpp:9-139, pinned by the
reference's own unit test (tests/test_engine.cpp:47-78, expected values in
tests/golden/block_manager_unit.json), the published FNV-1a 64 vectors and
MurmurHash3 finalizer inverse, and compared call by call on randomized
engine-style traces (src/engine/engine.cpp:176-205, :302-335)."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from ember_amd import BlockManager, EmberError

GOLDEN = json.loads((Path(__file__).parent / "golden" / "block_manager_unit.json").read_text())
PAGE = 16
IMPLS = {"product": BlockManager, "oracle": oracle.BlockManager}


@pytest.mark.parametrize("impl", IMPLS)
def test_reference_unit_test(impl):
    g = GOLDEN
    bm = IMPLS[impl](g["num_blocks"], g["prefix_caching"])
    toks = list(range(g["tokens_first"], g["tokens_first"] + g["tokens_count"]))
    mine, chain = [], 0
    for b in range(g["sealed_blocks"]):
        mine.append(bm.allocate())
        chain = bm.seal(mine[-1], chain, toks[b * PAGE:(b + 1) * PAGE])
    assert bm.available() == g["available_after_two_allocs"]
    hit = bm.match_prefix(toks)
    assert len(hit) == g["match_prefix_hits"]
    assert hit == mine and bm.refcount(mine[0]) == g["refcount_of_first_after_match"]
    bm.release_all(hit)
    bm.release_all(mine)
    assert bm.available() == g["available_after_release"]
    assert bm.cached() == g["cached_after_release"]
    again = bm.match_prefix(toks)
    assert len(again) == g["match_prefix_hits_again"]
    bm.release_all(again)
    other = list(toks)
    other[g["changed_token_index"]] = g["changed_token_value"]
    assert len(bm.match_prefix(other)) == g["hits_with_changed_token"]
    every = [bm.allocate() for _ in range(g["num_blocks"])]
    assert bm.allocate() == g["allocate_when_full"]
    assert bm.cached() == g["cached_after_taking_every_block"]
    assert bm.check() == ""
    bm.release_all(every)
    assert bm.check() == "" and bm.available() == g["available_at_end"]


def test_low_ids_first_and_lifo_reuse():
    for impl in IMPLS.values():
        bm = impl(5, True)
        assert [bm.allocate() for _ in range(3)] == [0, 1, 2]
        bm.release(1)
        assert bm.allocate() == 1  # a freed block goes on top of the stack
        bm.release_all([0, 2])     # released in reverse: 2, then 0 -> 0 comes out next
        assert [bm.allocate(), bm.allocate(), bm.allocate()] == [0, 2, 3]


# ---- the hash ----

def _fnv_bytes(s: bytes):
    return oracle.fnv1a_words(0, list(s))


def test_fnv1a_stage_matches_published_vectors():
    # FNV-1a 64 (Fowler/Noll/Vo) test vectors; one token per byte when tokens < 256 and parent = 0.
    assert _fnv_bytes(b"") == 0xCBF29CE484222325
    assert _fnv_bytes(b"a") == 0xAF63DC4C8601EC8C
    assert _fnv_bytes(b"foobar") == 0x85944171F73967E8


def _unfmix64(h):
    """Inverse of the MurmurHash3 fmix64 finalizer, with its published inverse constants."""
    M = (1 << 64) - 1
    h ^= h >> 33
    h = (h * 0x9CB4B2F8129337DB) & M
    h ^= h >> 33
    h = (h * 0x4F74430C22A54005) & M
    h ^= h >> 33
    return h


def test_fmix64_stage_inverts_with_published_constants(rng):
    assert oracle.fmix64(0) == 0
    for x in rng.integers(0, 2**63, 200, dtype=np.int64).tolist() + [1, 2**64 - 1]:
        assert _unfmix64(oracle.fmix64(int(x))) == int(x)


def test_block_hash_is_the_two_stages_and_never_zero(rng):
    for _ in range(200):
        parent = int(rng.integers(0, 2**63))
        toks = rng.integers(-(2**31), 2**31 - 1, PAGE).tolist()
        h = oracle.fmix64(oracle.fnv1a_words(parent, toks))
        assert oracle.BlockManager.block_hash(parent, toks) == (h or 1)
        assert BlockManager.block_hash(parent, toks) == (h or 1)  # product


# ---- randomized traces: product and oracle call for call ----

class Pair:
    """Applies every call to the product and the oracle and checks they answer alike."""

    def __init__(self, n, caching):
        self.p, self.o = BlockManager(n, caching), oracle.BlockManager(n, caching)

    def __getattr__(self, name):
        def call(*a):
            rp = getattr(self.p, name)(*a)
            ro = getattr(self.o, name)(*a)
            assert rp == ro, f"{name}{a}: product {rp} != oracle {ro}"
            return rp

        return call

    def audit(self):
        assert self.p.check() == "" and self.o.check() == ""
        assert self.p.states() == self.o.states()
        for f in ("available", "used", "cached", "hit_tokens", "lookup_tokens"):
            assert getattr(self.p, f)() == getattr(self.o, f)(), f


def _engine_trace(rng, n_blocks, n_seqs, steps, vocab, prefix_pool):
    """A miniature of the engine's block use: admission with match_prefix of all but the last token,
    ensure_blocks, sealing full blocks, preemption (release_all) of the newest sequence when out of blocks,
    finishing. A slot array plays FakeBackend (tests/fake_backend.hpp:57-74): every computed token is
    written to its page slot and every context is read back through the block table."""
    bm = Pair(n_blocks, True)
    slots = np.full(n_blocks * PAGE, -1, np.int64)
    seqs = []
    for _ in range(steps):
        if len(seqs) < n_seqs and rng.random() < 0.5:
            pre = prefix_pool[rng.integers(len(prefix_pool))]
            tail = rng.integers(2, vocab, rng.integers(1, 60)).tolist()
            seqs.append({"tokens": list(pre) + tail, "blocks": [], "computed": 0, "sealed": 0, "chain": 0,
                         "admitted": False})
        if not seqs:
            continue
        s = seqs[rng.integers(len(seqs))]
        if not s["admitted"]:
            got = bm.match_prefix(s["tokens"][:-1])
            s["blocks"], s["computed"], s["sealed"] = got, len(got) * PAGE, len(got)
            s["chain"] = 0
            for i in range(s["sealed"]):
                s["chain"] = BlockManager.block_hash(s["chain"], s["tokens"][i * PAGE:(i + 1) * PAGE])
            s["admitted"] = True
        n = min(len(s["tokens"]) - s["computed"], int(rng.integers(1, 40)))
        if n <= 0:  # generate one token
            s["tokens"].append(int(rng.integers(2, vocab)))
            n = 1
        need = (s["computed"] + n + PAGE - 1) // PAGE
        ok = True
        while len(s["blocks"]) < need:
            b = bm.allocate()
            if b >= 0:
                s["blocks"].append(b)
                continue
            # Out of blocks: preempt the newest other holder (engine.cpp:278-289), else this one.
            holders = [q for q in seqs if q is not s and q["blocks"]]
            victim = holders[-1] if holders else s
            bm.release_all(victim["blocks"])
            victim.update(blocks=[], computed=0, sealed=0, chain=0, admitted=False)
            if victim is s:
                ok = False
                break
        if not ok:
            continue
        for pos in range(s["computed"], s["computed"] + n):  # write, then read the whole context back
            slots[s["blocks"][pos // PAGE] * PAGE + pos % PAGE] = s["tokens"][pos]
        s["computed"] += n
        ctx = [slots[s["blocks"][p // PAGE] * PAGE + p % PAGE] for p in range(s["computed"])]
        assert ctx == s["tokens"][: s["computed"]], "a context read back through the block table differs"
        while (s["sealed"] + 1) * PAGE <= s["computed"]:
            chunk = s["tokens"][s["sealed"] * PAGE:(s["sealed"] + 1) * PAGE]
            s["chain"] = bm.seal(s["blocks"][s["sealed"]], s["chain"], chunk)
            s["sealed"] += 1
        if rng.random() < 0.08:  # finish
            bm.release_all(s["blocks"])
            seqs.remove(s)
        bm.audit()
        refs = np.zeros(n_blocks, int)
        for q in seqs:
            for b in q["blocks"]:
                refs[b] += 1
        assert all(bm.p.refcount(b) == refs[b] for b in range(n_blocks))
    for q in seqs:
        bm.release_all(q["blocks"])
    bm.audit()
    assert bm.p.used() == 0


@pytest.mark.parametrize("seed", range(6))
def test_engine_style_traces_match_oracle(seed):
    rng = np.random.default_rng(1000 + seed)
    prefixes = [rng.integers(2, 50, rng.integers(0, 80)).tolist() for _ in range(4)]
    _engine_trace(rng, n_blocks=int(rng.integers(12, 60)), n_seqs=8, steps=600, vocab=50, prefix_pool=prefixes)


def test_random_calls_match_oracle(rng):
    n = 24
    bm = Pair(n, True)
    held = []
    for _ in range(3000):
        r = rng.random()
        if r < 0.3:
            b = bm.allocate()
            if b >= 0:
                held.append(b)
        elif r < 0.45 and held:
            b = held.pop(int(rng.integers(len(held))))
            bm.release(b)
        elif r < 0.6 and held:
            b = held[int(rng.integers(len(held)))]
            toks = rng.integers(0, 4, PAGE).tolist()  # small vocab: identical blocks happen
            bm.seal(b, int(rng.integers(0, 3)), toks)
        elif r < 0.75:
            toks = rng.integers(0, 4, int(rng.integers(0, 70))).tolist()
            held += bm.match_prefix(toks)
        elif r < 0.85 and held and len(held) < 200:
            k = int(rng.integers(1, min(3, len(held)) + 1))
            sel = [held[i] for i in rng.choice(len(held), k, replace=False)]
            bm.share(sel)
            held += sel
        elif held:
            i = int(rng.integers(len(held)))
            nb = bm.copy_on_write(held[i])
            if nb >= 0:
                held[i] = nb
        bm.audit()
    bm.release_all(held)
    bm.audit()
    assert bm.p.available() == n


def test_copy_on_write_semantics():
    bm = BlockManager(6, True)
    a = bm.allocate()
    bm.share([a, a])                # three holders of a partial page
    assert bm.refcount(a) == 3
    b = bm.copy_on_write(a)         # a holder about to write gets its own page
    assert b != a and bm.refcount(a) == 2 and bm.refcount(b) == 1
    c = bm.copy_on_write(a)
    assert c not in (a, b) and bm.refcount(a) == 1
    assert bm.copy_on_write(a) == a  # the last holder writes in place
    assert bm.copy_on_write(b) == b
    assert bm.check() == ""
    bm.release_all([a, b, c])
    assert bm.available() == 6
    with pytest.raises(EmberError):
        bm.copy_on_write(a)          # not held
    with pytest.raises(EmberError):
        bm.share([a])
    # out of blocks: the reference stays held, -1 comes back
    full = BlockManager(2, True)
    x = full.allocate()
    full.share([x])
    y = full.allocate()
    assert full.copy_on_write(x) == -1 and full.refcount(x) == 2
    full.release_all([x, x, y])
    assert full.check() == ""


def test_errors_match_reference_behaviour():
    bm = BlockManager(4, True)
    with pytest.raises(EmberError):
        bm.release(0)                  # releasing a free block throws (block_manager.cpp:58)
    b = bm.allocate()
    with pytest.raises(EmberError):
        bm.seal(b, 0, list(range(15)))  # a block must be full to seal (:97)
    with pytest.raises(EmberError):
        BlockManager(0, True)           # no blocks (:10)
    nc = BlockManager(4, False)
    b = nc.allocate()
    h = nc.seal(b, 0, list(range(16)))
    assert h == BlockManager.block_hash(0, list(range(16))) and nc.cached() == 0
    assert nc.match_prefix(list(range(40))) == [] and nc.lookup_tokens() == 0


def test_large_pool_is_fast():
    """131,072 pages (2M tokens): allocation and release stay O(1) per call."""
    import time

    bm = BlockManager(131072, True)
    t0 = time.perf_counter()
    blocks = [bm.allocate() for _ in range(131072)]
    bm.release_all(blocks)
    dt = time.perf_counter() - t0
    assert bm.available() == 131072 and dt < 5.0
