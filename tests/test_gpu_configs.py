"""GPU parity at BASELINE.json's full workloads, one layer each, through the C++ path (HipPagedKv plan + layer)
and the product BlockManager, against the CPU oracle.

- config 3: 64 sequences sharing a 1024-token prefix (64 sealed pages, refcount 64), 4 x 512-token prefill
  chunks + 60 decodes, one forked pair copying its shared partial page on write;
- config 4: the 131,072-page pool, 256 sequences with contexts logU[512, 16384]; a decode step, then the
  newest 8 preempted and resumed by re-prefilling their whole contexts through the plan (prefill tiles) beside
  the other 248's decode;
- config 5: 64 sequences, contexts U[512, 4096], a q_len 5 verify (4 drafts + 1) with rollback to a seeded
  accepted count; verify equals sequential decode bit for bit.

Every page placement comes from the product BlockManager and is checked call for call against the oracle's
(bit-exact). Attention is checked against the oracle within 2e-3 (f16 KV) on a snapshot of the pages the step
reads (gpu_oracle); every slot the step does not write stays bit-identical, new V slots are bit-exact and new
K slots within one f16 ulp.
"""
import numpy as np
import pytest
import torch

import oracle
from ember_amd import BlockManager
from ember_amd.paged_kv import PagedKv, StepBatch
from gpu_oracle import check_pages_after, oracle_layer, snapshot, written_slots
from helpers import D, PAGE, rel_err

pytestmark = pytest.mark.gpu

H, KVH = 16, 8
W = (H + 2 * KVH) * D
EPS, THETA = 1e-6, 1e6
SEED = 20261005


class Pages:
    """The product BlockManager with the oracle's beside it: every call made on both, results compared."""

    def __init__(self, num_blocks, prefix_caching, rng):
        self.bm = BlockManager(num_blocks, prefix_caching)
        self.ref = oracle.BlockManager(num_blocks, prefix_caching)
        every = [self.allocate() for _ in range(num_blocks)]  # hand pages out in a seeded random order
        self.release_all([every[i] for i in rng.permutation(num_blocks)])

    def _both(self, name, *args):
        a, b = getattr(self.bm, name)(*args), getattr(self.ref, name)(*args)
        assert a == b, f"{name}{args[:1]}: product {a} != oracle {b}"
        return a

    def allocate(self):
        b = self._both("allocate")
        assert b >= 0, "the pool is exhausted"
        return b

    def release_all(self, blocks):
        self.bm.release_all(blocks)
        self.ref.release_all(blocks)
        assert self.bm.available() == self.ref.available()

    def seal(self, block, parent, tokens):
        return self._both("seal", block, parent, tokens)

    def match_prefix(self, tokens):
        return self._both("match_prefix", tokens)

    def share(self, blocks):
        self.bm.share(blocks)
        self.ref.share(blocks)

    def copy_on_write(self, block):
        return self._both("copy_on_write", block)

    def refcount(self, block):
        return self._both("refcount", block)

    def check(self):
        assert self.bm.check() == "" and self.ref.check() == ""
        assert self.bm.states() == self.ref.states()


def _norms(rng):
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    return qn, kn


def _fill_random(kv, layers, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    for layer in range(layers):
        for which in ("k", "v"):
            kv.pool_view(layer, which).normal_(generator=g)
    torch.cuda.synchronize()


def _run_layer(kv, layer, positions, query_start, tables, qkv16, qn, kn, device):
    """plan + one layer through the path; returns the outputs [T, H, D] as f32."""
    positions = np.asarray(positions, np.int32)
    query_start = np.asarray(query_start, np.int32)
    tables = np.asarray(tables, np.int32)
    T = positions.size
    if layer == 0:
        ctx = [int(positions[query_start[s + 1] - 1]) + 1 for s in range(tables.shape[0])]
        kv.plan(StepBatch(tokens=np.zeros(T, np.int32), positions=positions, query_start=query_start,
                          context_len=np.asarray(ctx, np.int32), block_tables=tables.reshape(-1),
                          max_blocks=tables.shape[1]))
    out = torch.full((T, H, D), float("nan"), dtype=torch.float16, device=device)
    kv.layer(layer, torch.from_numpy(qkv16).to(device), out, q_norm=torch.from_numpy(qn).to(device),
             k_norm=torch.from_numpy(kn).to(device))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _check_layer(kv, layer, positions, query_start, tables, qkv16, qn, kn, device, subset=None):
    """The step's layer on the GPU and on the oracle's snapshot; returns the GPU outputs."""
    positions = np.asarray(positions, np.int32)
    query_start = np.asarray(query_start, np.int32)
    tables = np.asarray(tables, np.int32)
    ctx = np.array([positions[query_start[s + 1] - 1] + 1 for s in range(tables.shape[0])])
    snap = snapshot(kv, layer, tables, (ctx + PAGE - 1) // PAGE)
    got = _run_layer(kv, layer, positions, query_start, tables, qkv16, qn, kn, device)
    want = oracle_layer(snap, qkv16.astype(np.float32), positions, query_start, n_heads=H, n_kv=KVH, q_norm=qn,
                        k_norm=kn, inv_freq=oracle.inv_freq(THETA, D), eps=EPS, subset=subset)
    sel = got if subset is None else got[np.asarray(subset)]
    assert np.isfinite(sel).all()
    err = rel_err(sel, want)
    assert err < 2e-3, f"layer {layer}: relative error {err:.2e}"
    check_pages_after(kv, layer, snap, written_slots(snap, positions, query_start))
    return got


def test_config3_mixed_step_full_size(device):
    """BASELINE config 3 at full size: 64 sequences share a 1024-token system prefix held in 64 sealed pages
    (prefix cache; refcount 64 once all are admitted); 4 prefill their own prompts in 512-token chunks (at chunk
    offsets 0..3, so contexts 1536..3072) on MFMA tiles; 60 decode one token with own contexts U[128, 2048] after
    the prefix; two of them are a fork sharing every page, partial last page included, so the step first copies
    that page on write (every layer, bit-exact). Two layers."""
    NSEQ, NPRE, PREFIX, CHUNK, NCHUNK, L = 64, 4, 1024, 512, 4, 2
    rng = np.random.default_rng(SEED + 3)
    own = rng.integers(128, 2049, NSEQ - NPRE)
    mb = (PREFIX + max(CHUNK * NCHUNK, int(own.max()) + 1) + PAGE) // PAGE + 1
    NB = PREFIX // PAGE + int(own.sum()) // PAGE + 3 * NSEQ + NPRE * CHUNK * NCHUNK // PAGE + 64
    pages = Pages(NB, True, rng)
    kv = PagedKv(n_layers=L, n_heads=H, n_kv_heads=KVH, rms_eps=EPS, rope_theta=THETA, max_position=mb * PAGE,
                 num_blocks=NB, max_batch_tokens=NPRE * CHUNK + NSEQ, max_seqs=NSEQ, dtype=torch.float16)
    _fill_random(kv, L, SEED + 3)
    prefix = rng.integers(0, 150000, PREFIX).astype(np.int32)
    prefix_blocks, parent = [], 0
    for i in range(PREFIX // PAGE):  # the prefix, computed once and sealed into the prefix cache
        b = pages.allocate()
        parent = pages.seal(b, parent, prefix[i * PAGE:(i + 1) * PAGE])
        prefix_blocks.append(b)
    pages.release_all(prefix_blocks)  # held by the cache until a sequence matches it
    blocks = [[] for _ in range(NSEQ)]
    ctx = np.zeros(NSEQ, np.int64)

    def admit(s, upto):
        got = pages.match_prefix(np.concatenate([prefix, np.zeros(1, np.int32)]))
        assert got == prefix_blocks, "the prefix cache missed"
        blocks[s] = list(got)
        while len(blocks[s]) * PAGE < upto:
            blocks[s].append(pages.allocate())

    for s in range(NPRE, NSEQ - 1):
        ctx[s] = PREFIX + int(own[s - NPRE])
        admit(s, ctx[s] + 1)
    fork, src = NSEQ - 1, NSEQ - 2  # the fork shares every page of its source, partial last page included
    ctx[src] = PREFIX + int(own[src - NPRE]) | 1  # an odd context: the last page is partial
    while len(blocks[src]) * PAGE < ctx[src] + 1:
        blocks[src].append(pages.allocate())
    pages.share(blocks[src])
    blocks[fork], ctx[fork] = list(blocks[src]), ctx[src]
    chunk_of = [0, 1, 2, 3]
    for s in range(NPRE):
        admit(s, PREFIX + CHUNK * NCHUNK)
        ctx[s] = PREFIX + CHUNK * chunk_of[s]
    assert pages.refcount(prefix_blocks[0]) == NSEQ and pages.refcount(prefix_blocks[-1]) == NSEQ
    last_page = int(ctx[src]) // PAGE
    assert pages.refcount(blocks[src][last_page]) == 2

    # copy-on-write before the first write into the shared partial page (the fork writes; the source is then
    # the page's only holder and writes in place)
    before = [[kv.pool_view(l, w)[blocks[src][last_page]].clone() for w in ("k", "v")] for l in range(L)]
    nb = pages.copy_on_write(blocks[fork][last_page])
    assert nb >= 0 and nb != blocks[src][last_page]
    kv.copy_blocks([blocks[fork][last_page]], [nb])
    blocks[fork][last_page] = nb
    assert pages.copy_on_write(blocks[src][last_page]) == blocks[src][last_page]
    torch.cuda.synchronize()
    for l in range(L):
        for i, w in enumerate(("k", "v")):
            assert torch.equal(kv.pool_view(l, w)[nb].view(torch.int16), before[l][i].view(torch.int16))

    tables = np.zeros((NSEQ, mb), np.int32)
    for s in range(NSEQ):
        tables[s, :len(blocks[s])] = blocks[s]
    pos, qs = [], [0]
    for s in range(NSEQ):
        n = CHUNK if s < NPRE else 1
        pos.append(np.arange(ctx[s], ctx[s] + n))
        qs.append(qs[-1] + n)
    pos = np.concatenate(pos).astype(np.int32)
    T = pos.size
    assert T == NPRE * CHUNK + NSEQ - NPRE
    # every decode token, and every 7th prefill token plus each chunk's last
    subset = sorted(set(range(NPRE * CHUNK, T)) | set(range(0, NPRE * CHUNK, 7)) |
                    {(s + 1) * CHUNK - 1 for s in range(NPRE)})
    for l in range(L):
        qn, kn = _norms(rng)
        qkv = rng.standard_normal((T, W)).astype(np.float16)
        _check_layer(kv, l, pos, qs, tables, qkv, qn, kn, device, subset=subset)
    runs, tiles, splits, fused = kv.plan_info()
    assert tiles == NPRE * CHUNK // 64 and runs == NSEQ - NPRE and not fused
    # the shared prefix was never written (check_pages_after: slots outside the step's writes are unchanged),
    # and after the step every sequence still holds it
    assert pages.refcount(prefix_blocks[0]) == NSEQ
    pages.check()


def test_config4_preempt_and_reprefill_full_size(device):
    """BASELINE config 4 at full size, one layer: the 131,072-page pool (2,097,152 tokens), 256 sequences with
    contexts logU[512, 16384]. Step 1 decodes one token for each. Then the newest 8 are preempted (pages back to
    the pool) and resumed in step 2 by re-prefilling their whole contexts through the plan (runs of >= 16 tokens:
    MFMA prefill tiles) beside the other 248's decode. Both steps against the oracle."""
    POOL, NSEQ, PRE = 131072, 256, 8
    rng = np.random.default_rng(SEED + 4)
    ctx = np.exp(rng.uniform(np.log(512), np.log(16384), NSEQ)).astype(np.int64)
    mb = (int(ctx.max()) + 2 * PAGE) // PAGE + 1
    pages = Pages(POOL, False, rng)
    resumed_tokens = int(np.sort(ctx)[-PRE:].sum()) + PRE * 2
    kv = PagedKv(n_layers=1, n_heads=H, n_kv_heads=KVH, rms_eps=EPS, rope_theta=THETA, max_position=mb * PAGE,
                 num_blocks=POOL, max_batch_tokens=NSEQ + resumed_tokens, max_seqs=NSEQ, dtype=torch.float16)
    _fill_random(kv, 1, SEED + 4)
    blocks = [[] for _ in range(NSEQ)]

    def ensure(s, upto):
        while len(blocks[s]) * PAGE < upto:
            blocks[s].append(pages.allocate())

    def tables_of(seqs):
        t = np.zeros((len(seqs), mb), np.int32)
        for i, s in enumerate(seqs):
            t[i, :len(blocks[s])] = blocks[s]
        return t

    qn, kn = _norms(rng)
    # step 1: every sequence decodes one token (fused append + attention, 33 splits at 16k)
    for s in range(NSEQ):
        ensure(s, int(ctx[s]) + 1)
    seqs = list(range(NSEQ))
    qkv = rng.standard_normal((NSEQ, W)).astype(np.float16)
    _check_layer(kv, 0, ctx.astype(np.int32), np.arange(NSEQ + 1), tables_of(seqs), qkv, qn, kn, device)
    assert kv.fused()
    ctx += 1
    # preempt the newest 8: their pages go back to the pool
    newest = seqs[-PRE:]
    for s in newest:
        pages.release_all(blocks[s])
        blocks[s] = []
    running = seqs[:-PRE]
    # step 2: the 248 running decode, the 8 resumed re-prefill their whole contexts (positions 0..ctx-1)
    order = running + newest
    pos, qs = [], [0]
    for s in order:
        if s in newest:
            ensure(s, int(ctx[s]))
            pos.append(np.arange(0, ctx[s]))
        else:
            ensure(s, int(ctx[s]) + 1)
            pos.append(np.array([ctx[s]]))
        qs.append(qs[-1] + pos[-1].size)
    pos = np.concatenate(pos).astype(np.int32)
    T = pos.size
    qkv = rng.standard_normal((T, W)).astype(np.float16)
    n_dec = len(running)
    pre = np.arange(n_dec, T)
    subset = sorted(set(range(n_dec)) | set(pre[::61].tolist()) | {qs[i + 1] - 1 for i in range(n_dec, len(order))})
    _check_layer(kv, 0, pos, qs, tables_of(order), qkv, qn, kn, device, subset=subset)
    runs, tiles, splits, fused = kv.plan_info()
    assert runs == n_dec and tiles == sum(-(-int(ctx[s]) // 64) for s in newest) and not fused
    pages.check()
    kv.close()


def test_config5_verify_rollback_full_size(device):
    """BASELINE config 5 at full size, one layer: 64 sequences with cached contexts U[512, 4096]; one step
    appends the last accepted token and 4 drafts per sequence and attends with q_len 5, causal inside the
    window (one fused launch); it matches the oracle, and every accepted row equals plain sequential decode of
    the same tokens bit for bit. Rollback to accepted U{0..4}: the next token goes to position c + accepted + 1
    in both worlds, with bit-identical outputs and bit-identical valid slots."""
    B, Q = 64, 5
    rng = np.random.default_rng(SEED + 5)
    c = rng.integers(512, 4097, B).astype(np.int64)
    mb = int((c.max() + Q + 2 + PAGE) // PAGE)
    NB = int(((c + Q + 2 + PAGE) // PAGE).sum()) + 16
    pages = Pages(NB, False, rng)
    tables = np.zeros((B, mb), np.int32)
    for s in range(B):
        for p in range(int((c[s] + Q + 1 + PAGE - 1) // PAGE)):
            tables[s, p] = pages.allocate()
    mk = lambda: PagedKv(n_layers=1, n_heads=H, n_kv_heads=KVH, rms_eps=EPS, rope_theta=THETA,  # noqa: E731
                         max_position=mb * PAGE, num_blocks=NB, max_batch_tokens=B * Q, max_seqs=B,
                         dtype=torch.float16)
    A, C = mk(), mk()  # verify world, sequential world, identical pools
    _fill_random(A, 1, SEED + 5)
    for w in ("k", "v"):
        C.pool_view(0, w).copy_(A.pool_view(0, w))
    torch.cuda.synchronize()
    qn, kn = _norms(rng)
    win = rng.standard_normal((B, Q, W)).astype(np.float16)
    pos = (c[:, None] + np.arange(Q)[None, :]).reshape(-1).astype(np.int32)
    qs = np.arange(B + 1) * Q
    va = _check_layer(A, 0, pos, qs, tables, win.reshape(-1, W), qn, kn, device).reshape(B, Q, H, D)
    assert A.fused(), "one 5-token run per sequence runs fused"
    accepted = rng.integers(0, Q, B)
    seq_out = np.zeros_like(va)
    for i in range(Q):  # sequential decode of the accepted window tokens, one step per position
        live = [s for s in range(B) if i <= accepted[s]]
        o = _run_layer(C, 0, (c[live] + i).astype(np.int32), np.arange(len(live) + 1), tables[live],
                       np.stack([win[s, i] for s in live]), qn, kn, device)
        for j, s in enumerate(live):
            seq_out[s, i] = o[j]
    for s in range(B):
        a, b = va[s, :accepted[s] + 1], seq_out[s, :accepted[s] + 1]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"sequence {s}: verify != sequential decode"
    npos = (c + accepted + 1).astype(np.int32)
    nxt = rng.standard_normal((B, W)).astype(np.float16)
    oa = _check_layer(A, 0, npos, np.arange(B + 1), tables, nxt, qn, kn, device)
    oc = _run_layer(C, 0, npos, np.arange(B + 1), tables, nxt, qn, kn, device)
    assert np.array_equal(oa.view(np.uint32), oc.view(np.uint32))
    ka, vka = A.pool_view(0, "k").cpu().numpy(), A.pool_view(0, "v").cpu().numpy()
    kc, vkc = C.pool_view(0, "k").cpu().numpy(), C.pool_view(0, "v").cpu().numpy()
    for s in range(B):
        for p in range(int(npos[s]) + 1):  # every slot that is valid after the rollback
            b, sl = tables[s, p // PAGE], p % PAGE
            assert np.array_equal(ka[b, :, sl].view(np.uint16), kc[b, :, sl].view(np.uint16))
            assert np.array_equal(vka[b, :, sl].view(np.uint16), vkc[b, :, sl].view(np.uint16))
    pages.check()
