"""GPU parity of the whole paged-KV path (C++ HipPagedKv + BlockManager through the C ABI) against the
CPU oracle, on the BASELINE.json workloads at test scale.

Tolerances: slots and pages bit-exact; attention within 2e-3 (f16 KV) / 1e-5 (f32 KV) relative error
(helpers.rel_err), against the oracle's f32 CPU path fed the same activations.
"""
import numpy as np
import pytest
import torch

import oracle
from ember_amd import BlockManager, EmberError
from ember_amd.paged_kv import PagedKv, StepBatch
from gpu_oracle import oracle_layer, snapshot
from helpers import D, PAGE, rel_err

pytestmark = pytest.mark.gpu

H, KVH = 16, 8
W = (H + 2 * KVH) * D
EPS, THETA = 1e-6, 1e6


class World:
    """The GPU path and the oracle side by side, driven with identical steps."""

    def __init__(self, device, dtype, num_blocks, n_layers=1, max_position=8192, max_batch_tokens=2048, seed=0,
                 n_heads=H, n_kv=KVH, max_seqs=64):
        self.dev, self.dtype, self.NB, self.L = device, dtype, num_blocks, n_layers
        self.H, self.KVH, self.W = n_heads, n_kv, (n_heads + 2 * n_kv) * D
        self.kv = PagedKv(n_layers=n_layers, n_heads=n_heads, n_kv_heads=n_kv, rms_eps=EPS, rope_theta=THETA,
                          max_position=max_position, num_blocks=num_blocks, max_batch_tokens=max_batch_tokens,
                          max_seqs=max_seqs, dtype=dtype)
        r = np.random.default_rng(seed)
        self.qn = [(1 + 0.1 * r.standard_normal(D)).astype(np.float32) for _ in range(n_layers)]
        self.kn = [(1 + 0.1 * r.standard_normal(D)).astype(np.float32) for _ in range(n_layers)]
        self.qn_d = [torch.from_numpy(a).to(device) for a in self.qn]
        self.kn_d = [torch.from_numpy(a).to(device) for a in self.kn]
        # the oracle keeps f32 pools with the same number of blocks (+ the spare, never read)
        self.ko = [np.zeros((num_blocks + 1, n_kv, PAGE, D), np.float32) for _ in range(n_layers)]
        self.vo = [np.zeros_like(self.ko[0]) for _ in range(n_layers)]
        self.inv = oracle.inv_freq(THETA, D)

    def step(self, positions, query_start, tables, qkv_layers, check=True, oracle_tables=None):
        """One step: plan, then per layer append + attention. qkv_layers: [L][T, W] f32 values (f16-exact
        when the pools are f16). oracle_tables: the oracle's own block tables (default: the GPU's). Returns
        (gpu outputs, oracle outputs or None when not check) per layer, f32 arrays [T, H, D]."""
        positions = np.asarray(positions, np.int32)
        query_start = np.asarray(query_start, np.int32)
        tables = np.asarray(tables, np.int32)
        otab = tables if oracle_tables is None else np.asarray(oracle_tables, np.int32)
        S, T = tables.shape[0], positions.size
        ctx = [int(positions[query_start[s + 1] - 1]) + 1 for s in range(S)]
        self.kv.plan(StepBatch(tokens=[0] * T, positions=positions.tolist(), query_start=query_start.tolist(),
                               context_len=ctx, block_tables=tables.reshape(-1).tolist(), max_blocks=tables.shape[1]))
        res = []
        for layer in range(self.L):
            qkv = qkv_layers[layer]
            qkv_d = torch.from_numpy(qkv).to(self.dev, self.dtype)
            out = torch.full((T, self.H, D), float("nan"), dtype=self.dtype, device=self.dev)
            self.kv.layer(layer, qkv_d, out, q_norm=self.qn_d[layer], k_norm=self.kn_d[layer])
            q_ref = oracle.append_layer(qkv, positions, query_start, otab, self.ko[layer], self.vo[layer],
                                        n_heads=self.H, n_kv=self.KVH, inv_freq_=self.inv, eps=EPS,
                                        q_norm=self.qn[layer], k_norm=self.kn[layer], num_blocks=self.NB + 1,
                                        kv_f16=False)
            want = None
            if check:
                want = oracle.attention_layer(q_ref, positions, query_start, otab, self.ko[layer], self.vo[layer],
                                              n_heads=self.H, n_kv=self.KVH, num_blocks=self.NB + 1, kv_f16=False,
                                              threads=8)
            torch.cuda.synchronize()
            res.append((out.float().cpu().numpy(), want))
        return res

    def pools(self, layer):
        return (self.kv.pool_view(layer, "k").float().cpu().numpy(), self.kv.pool_view(layer, "v").float().cpu().numpy())

    @property
    def tol(self):
        return 2e-3 if self.dtype == torch.float16 else 1e-5


def _acts(rng, T, L, f16, width=W):
    a = [rng.standard_normal((T, width)).astype(np.float32) for _ in range(L)]
    return [x.astype(np.float16).astype(np.float32) for x in a] if f16 else a


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_config1_prefill_then_decode(rng, device, dtype):
    """one Qwen3-0.6B-shaped layer, batch 1, a 512-token prefill into 16-token pages,
    then 128 decode steps; the block table is the first 40 entries of a seeded permutation of 4096 pages."""
    f16 = dtype == torch.float16
    w = World(device, dtype, num_blocks=4096, max_position=640)
    table = rng.permutation(4096)[:40].astype(np.int32)[None, :]
    outs = w.step(np.arange(512), [0, 512], table, _acts(rng, 512, 1, f16))
    worst = rel_err(*outs[0])
    for pos in range(512, 640):
        outs = w.step([pos], [0, 1], table, _acts(rng, 1, 1, f16))
        worst = max(worst, rel_err(*outs[0]))
    assert worst < w.tol, f"worst relative error {worst:.2e}"
    # page placement: exactly the table's 40 pages hold data, slot for slot
    kg, vg = w.pools(0)
    written_g = np.abs(kg).sum(axis=(1, 3)) > 0  # [NB+1, 16] per (block, slot), any kv head
    written_o = np.abs(w.ko[0]).sum(axis=(1, 3)) > 0
    assert np.array_equal(written_g, written_o)
    assert set(np.nonzero(written_g.any(axis=1))[0]) == set(table[0].tolist())
    tolk = 2e-3 if f16 else 1e-5
    assert rel_err(kg[table[0]], w.ko[0][table[0]]) < tolk and rel_err(vg[table[0]], w.vo[0][table[0]]) < tolk


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_uneven_chunks_at_block_offset_3(device, dtype):
    """The reference's uneven-chunk check (tests/test_model.cpp:124-157) at the attention layer: a 700-token
    prompt (seeded N(0,1) activations) run in chunks of 300, 37 (ending in the middle of a page) and 363 (64-token
    tiles and partial tiles), then 8 decode steps. As there, the GPU sequence sits on consecutive blocks from 3
    (SingleSequence(gpu, 3), tests/model_helpers.hpp:13) and the oracle's from 0: different physical blocks on
    purpose. Every token of every step within 2e-3 (f16) / 1e-5 (f32); the pages match slot for slot."""
    f16 = dtype == torch.float16
    rng = np.random.default_rng(12345)
    w = World(device, dtype, num_blocks=64, max_position=1024)
    n_pages = (700 + 8 + PAGE - 1) // PAGE
    gtab = (3 + np.arange(n_pages, dtype=np.int32))[None, :]
    otab = np.arange(n_pages, dtype=np.int32)[None, :]
    length = 0
    for chunk in (300, 37, 363):
        (got, want), = w.step(np.arange(length, length + chunk), [0, chunk], gtab, _acts(rng, chunk, 1, f16),
                              oracle_tables=otab)
        assert rel_err(got, want) < w.tol, f"chunk ending at {length + chunk}"
        length += chunk
    for _ in range(8):
        (got, want), = w.step([length], [0, 1], gtab, _acts(rng, 1, 1, f16), oracle_tables=otab)
        assert rel_err(got, want) < w.tol, f"decode at {length}"
        length += 1
    kg, vg = w.pools(0)
    tolk = 2e-3 if f16 else 1e-5
    assert rel_err(kg[gtab[0]], w.ko[0][otab[0]]) < tolk and rel_err(vg[gtab[0]], w.vo[0][otab[0]]) < tolk
    assert not np.abs(kg[:3]).any() and not np.abs(kg[3 + n_pages:]).any(), "a block outside the table was written"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_mixed_step(rng, device, dtype):
    """Prompt chunks and decodes in one step (continuous batching), 2 layers."""
    f16 = dtype == torch.float16
    w = World(device, dtype, num_blocks=600, n_layers=2)
    perm = rng.permutation(600).astype(np.int32)
    ctx0 = [0, 100, 1030, 0, 16, 511]          # cached before the step
    new = [40, 1, 1, 16, 1, 37]                # new tokens this step
    tables = np.zeros((6, 100), np.int32)
    at = 0
    for s in range(6):
        n_pages = (ctx0[s] + new[s] + PAGE - 1) // PAGE
        tables[s, :n_pages] = perm[at:at + n_pages]
        at += n_pages
    # fill the cached contexts through the path itself (prefill steps), then the mixed step
    for s in range(6):
        if ctx0[s]:
            w.step(np.arange(ctx0[s]), [0, ctx0[s]], tables[s:s + 1], _acts(rng, ctx0[s], 2, f16), check=False)
    pos, qs = [], [0]
    for s in range(6):
        pos += list(range(ctx0[s], ctx0[s] + new[s]))
        qs.append(len(pos))
    res = w.step(pos, qs, tables, _acts(rng, len(pos), 2, f16))
    for got, want in res:
        assert rel_err(got, want) < w.tol


@pytest.mark.parametrize("heads", [(32, 8), (24, 8), (64, 8)], ids=["G4", "G3", "G8"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_group_sizes_verify_chunk_and_decode(rng, device, dtype, heads):
    """Wider GQA groups (Qwen3-4B/8B have 32 query heads over 8 kv heads, G = 4; also G = 3 and G = 8): a
    decode work-group holds at most 16 query rows, so the planner cuts runs at min(8, 16 / G) tokens. One step
    with a 5-token verify run, a 12-token chunk (decode runs at every G), a 40-token prompt chunk (prefill tiles
    for f16, decode runs for f32) and a single decode, checked against the oracle."""
    f16 = dtype == torch.float16
    n_heads, n_kv = heads
    w = World(device, dtype, num_blocks=400, n_heads=n_heads, n_kv=n_kv, max_position=2048)
    perm = rng.permutation(400).astype(np.int32)
    ctx0 = [700, 300, 0, 1100]   # cached before the step
    new = [5, 12, 40, 1]         # new tokens this step
    tables = np.zeros((4, 80), np.int32)
    at = 0
    for s in range(4):
        n_pages = (ctx0[s] + new[s] + PAGE - 1) // PAGE
        tables[s, :n_pages] = perm[at:at + n_pages]
        at += n_pages
    for s in range(4):
        if ctx0[s]:
            w.step(np.arange(ctx0[s]), [0, ctx0[s]], tables[s:s + 1], _acts(rng, ctx0[s], 1, f16, w.W), check=False)
    pos, qs = [], [0]
    for s in range(4):
        pos += list(range(ctx0[s], ctx0[s] + new[s]))
        qs.append(len(pos))
    (got, want), = w.step(pos, qs, tables, _acts(rng, len(pos), 1, f16, w.W))
    assert np.isfinite(got).all()
    assert rel_err(got, want) < w.tol
    runs, tiles, _, fused = w.kv.plan_info()
    cap = min(8, 16 // (n_heads // n_kv))
    want_runs = sum(-(-n // cap) for n in new if not (f16 and n >= 16))
    assert runs == want_runs and tiles == (1 if f16 else 0) and not fused


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_verify_rollback_equals_sequential_decode(rng, device, dtype):
    """BASELINE config 5 at test scale: 4 drafts + the last token verified in one step (q_len 5, causal
    inside the window), rollback with accepted count ~U{0..4}; outputs and the slots that stay valid are
    bit-identical to plain one-token-per-step decoding."""
    f16 = dtype == torch.float16
    B, k = 8, 4
    c = rng.integers(512, 1500, B)              # cached context per sequence
    NB = int(((c + k + 2 + PAGE) // PAGE).sum()) + 8
    perm = rng.permutation(NB).astype(np.int32)
    mb = int((c.max() + k + 2 + PAGE) // PAGE)
    tables = np.zeros((B, mb), np.int32)
    at = 0
    for s in range(B):
        n_pages = int((c[s] + k + 2 + PAGE - 1) // PAGE)
        tables[s, :n_pages] = perm[at:at + n_pages]
        at += n_pages
    A = World(device, dtype, num_blocks=NB, max_position=mb * PAGE)   # verify world
    C = World(device, dtype, num_blocks=NB, max_position=mb * PAGE)   # sequential world
    for s in range(B):  # identical cached prefixes in both worlds
        acts = _acts(rng, int(c[s]), 1, f16)
        A.step(np.arange(c[s]), [0, c[s]], tables[s:s + 1], acts, check=False)
        C.step(np.arange(c[s]), [0, c[s]], tables[s:s + 1], acts, check=False)
    win = _acts(rng, B * (k + 1), 1, f16)[0].reshape(B, k + 1, W)
    pos = np.concatenate([np.arange(c[s], c[s] + k + 1) for s in range(B)])
    qs = np.arange(0, B * (k + 1) + 1, k + 1)
    (va, _), = A.step(pos, qs, tables, [win.reshape(-1, W)])
    accepted = rng.integers(0, k + 1, B)
    # the sequential world decodes only the accepted window tokens, one step per position
    seq_out = np.zeros_like(va).reshape(B, k + 1, H, D)
    for i in range(k + 1):
        live = [s for s in range(B) if i <= accepted[s]]
        (o, _), = C.step([c[s] + i for s in live], np.arange(len(live) + 1), tables[live],
                         [np.stack([win[s, i] for s in live])])
        for j, s in enumerate(live):
            seq_out[s, i] = o[j]
    va = va.reshape(B, k + 1, H, D)
    for s in range(B):
        a = va[s, :accepted[s] + 1]
        b = seq_out[s, :accepted[s] + 1]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"sequence {s}: verify != sequential decode"
    # after rollback the next token goes to position c + accepted + 1 in both worlds
    nxt = _acts(rng, B, 1, f16)[0]
    npos = [int(c[s] + accepted[s] + 1) for s in range(B)]
    (oa, wa), = A.step(npos, np.arange(B + 1), tables, [nxt])
    (oc, _), = C.step(npos, np.arange(B + 1), tables, [nxt])
    assert np.array_equal(oa.view(np.uint32), oc.view(np.uint32))
    assert rel_err(oa, wa) < A.tol
    ka, va_ = A.pools(0)
    kc, vc = C.pools(0)
    for s in range(B):
        for p in range(npos[s] + 1):  # every slot that is valid after the rollback
            b, sl = tables[s, p // PAGE], p % PAGE
            assert np.array_equal(ka[b, :, sl], kc[b, :, sl]) and np.array_equal(va_[b, :, sl], vc[b, :, sl])


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_fork_copy_on_write(rng, device, dtype):
    """BASELINE config 3's sharing at test scale: sequences share a system prefix of full sealed pages
    (refcounted via match_prefix) plus a partial last page (via share, a fork); the first write into the
    shared partial page copies it (copy_on_write + a device page copy), bit-exactly, over every layer."""
    f16 = dtype == torch.float16
    NB, L, n_children = 64, 3, 6
    prefix_len = 4 * PAGE + 5                 # 4 full pages + 5 tokens in a partial page
    bm = BlockManager(NB, True)
    w = World(device, dtype, num_blocks=NB, n_layers=L, max_position=256)
    tokens = rng.integers(2, 1000, prefix_len).tolist()
    parent = [bm.allocate() for _ in range(5)]
    chain = 0
    for i in range(4):
        chain = bm.seal(parent[i], chain, tokens[i * PAGE:(i + 1) * PAGE])
    tab = np.zeros((1, 8), np.int32)
    tab[0, :5] = parent
    w.step(np.arange(prefix_len), [0, prefix_len], tab, _acts(rng, prefix_len, L, f16), check=False)
    # children: the sealed pages by prefix match, the partial page by fork
    kids = []
    for _ in range(n_children):
        got = bm.match_prefix(tokens[:-1])
        assert got == parent[:4]
        bm.share([parent[4]])
        kids.append(got + [parent[4]])
    for b in parent[:4]:
        assert bm.refcount(b) == 1 + n_children
    assert bm.refcount(parent[4]) == 1 + n_children
    k_before = [w.pools(layer) for layer in range(L)]
    # every holder about to write position prefix_len: copy-on-write
    seqs = kids + [list(parent)]
    src, dst = [], []
    for blocks in seqs:
        nb = bm.copy_on_write(blocks[4])
        assert nb >= 0
        if nb != blocks[4]:
            src.append(blocks[4])
            dst.append(nb)
            blocks[4] = nb
    assert len(src) == n_children and bm.refcount(parent[4]) == 1  # the last holder writes in place
    w.kv.copy_blocks(src, dst)
    for o in range(L):  # mirror the copies in the oracle's pools
        for s_, d_ in zip(src, dst):
            w.ko[o][d_] = w.ko[o][s_]
            w.vo[o][d_] = w.vo[o][s_]
    torch.cuda.synchronize()
    for layer in range(L):
        kg, vg = w.pools(layer)
        k0, v0 = k_before[layer]
        for s_, d_ in zip(src, dst):  # page copies are bit-exact, every layer, K and V
            assert np.array_equal(kg[d_].view(np.uint32), k0[s_].view(np.uint32))
            assert np.array_equal(vg[d_].view(np.uint32), v0[s_].view(np.uint32))
    tables = np.zeros((len(seqs), 8), np.int32)
    for i, blocks in enumerate(seqs):
        tables[i, :5] = blocks
    res = w.step([prefix_len] * len(seqs), np.arange(len(seqs) + 1), tables, _acts(rng, len(seqs), L, f16))
    for got, want in res:
        assert rel_err(got, want) < w.tol
    kg, _ = w.pools(0)
    k0, _ = k_before[0]
    slot = prefix_len % PAGE
    for i, blocks in enumerate(seqs):  # each sequence's new token landed in its own page
        assert not np.array_equal(kg[blocks[4], :, slot], k0[parent[4], :, slot])
        assert np.array_equal(kg[blocks[4], :, :slot].view(np.uint32), k0[parent[4], :, :slot].view(np.uint32))
    for b in parent[:4]:  # shared sealed pages were never written
        assert np.array_equal(kg[b].view(np.uint32), k0[b].view(np.uint32))
    for blocks in seqs:
        bm.release_all(blocks)
    assert bm.check() == "" and bm.used() == 0 and bm.cached() == 4


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_decode_graph_equals_plan_and_layer(rng, device, dtype):
    """Decode steps run as replayed hipGraphs (padded to a token bucket and a block-table width bucket,
    padding tokens on the spare block) leave the same outputs and pools, to the bit, as plan + layer: the
    same graph replayed step after step with eager work in between, and new graphs when the batch moves
    to another bucket. Only the spare block differs (the padding writes there and nowhere else). Every
    replay's outputs are also checked against the oracle (2e-3 f16, 1e-5 f32) on a snapshot of the pages
    the step reads. A graph is captured once per (token bucket, width bucket) and then relaunched: the
    first bucket runs for more steps than the planner's staging ring has buffers, so its kept graph is
    launched with step integers staged through every buffer of the ring."""
    L, NB, maxpos = 2, 700, 2048
    mk = lambda: PagedKv(n_layers=L, n_heads=H, n_kv_heads=KVH, rms_eps=EPS, rope_theta=THETA,  # noqa: E731
                         max_position=maxpos, num_blocks=NB, max_batch_tokens=64, max_seqs=64, dtype=dtype)
    ga, eb = mk(), mk()
    qn = [torch.from_numpy((1 + 0.1 * rng.standard_normal(D)).astype(np.float32)).to(device) for _ in range(L)]
    kn = [torch.from_numpy((1 + 0.1 * rng.standard_normal(D)).astype(np.float32)).to(device) for _ in range(L)]
    qkv = [torch.zeros((64, W), dtype=dtype, device=device) for _ in range(L)]  # fixed buffers: graphs keep them
    out_g = [torch.zeros((64, H, D), dtype=dtype, device=device) for _ in range(L)]
    out_e = [torch.zeros((64, H, D), dtype=dtype, device=device) for _ in range(L)]
    io = [(qkv[l], out_g[l], qn[l], kn[l], None) for l in range(L)]
    ctx = [int(c) for c in rng.integers(1, 240, 9)]  # tokens cached per sequence
    blocks = [[] for _ in ctx]
    free = list(rng.permutation(NB))
    # active sequences per step: same bucket (replays) for 11 steps, then 7 -> bucket 8, 3 -> bucket 3; contexts
    # grow past 256 tokens (width bucket 16 -> 64 blocks) on the way
    active_per_step = [5] * 11 + [7, 7, 3, 3, 9]
    buckets = (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 40, 48, 56, 64)

    def width_bucket(w):  # HipPagedKv::width_bucket: 16 * 4^k blocks, at most the table's width
        b = 16
        while b < w:
            b *= 4
        return min(b, maxpos // PAGE)

    keys = set()
    for step, n_act in enumerate(active_per_step):
        seqs = list(range(n_act))
        if step == 12:
            for s in seqs:
                ctx[s] += 200  # jump: as if many steps had passed
        for s in seqs:
            while len(blocks[s]) * PAGE < ctx[s] + 1:
                blocks[s].append(int(free.pop()))
        mb = max(len(blocks[s]) for s in seqs)
        tables = np.zeros((n_act, mb), np.int32)
        for i, s in enumerate(seqs):
            tables[i, :len(blocks[s])] = blocks[s]
        pos = np.array([ctx[s] for s in seqs], np.int32)
        batch = StepBatch(tokens=[0] * n_act, positions=pos, query_start=np.arange(n_act + 1, dtype=np.int32),
                          context_len=pos + 1, block_tables=tables.reshape(-1), max_blocks=mb)
        acts = _acts(rng, n_act, L, dtype == torch.float16)
        for l in range(L):
            qkv[l][:n_act] = torch.from_numpy(acts[l]).to(device, dtype)
        # the oracle's view of the pages this step reads, before the step (both worlds hold the same pages)
        snaps = [snapshot(eb, l, tables, (pos + PAGE) // PAGE) for l in range(L)]
        keys.add((next(b for b in buckets if b >= n_act), width_bucket(mb)))
        assert ga.decode_graph(batch, io)
        assert ga.graph_captures() == len(keys), f"step {step}: one capture per bucket pair, relaunched after"
        eb.plan(batch)
        for l in range(L):
            eb.layer(l, qkv[l][:n_act], out_e[l][:n_act], q_norm=qn[l], k_norm=kn[l])
        torch.cuda.synchronize()
        bits = lambda t: t.cpu().numpy().view(np.uint16 if dtype == torch.float16 else np.uint32)  # noqa: E731
        for l in range(L):
            want = oracle_layer(snaps[l], acts[l], pos, np.arange(n_act + 1), n_heads=H, n_kv=KVH,
                                q_norm=qn[l].cpu().numpy(), k_norm=kn[l].cpu().numpy(), inv_freq=oracle.inv_freq(THETA, D),
                                eps=EPS, threads=8)
            tol = 2e-3 if dtype == torch.float16 else 1e-5
            assert rel_err(out_g[l][:n_act].float().cpu().numpy(), want) < tol, f"step {step} layer {l}: graph vs oracle"
            assert np.array_equal(bits(out_g[l][:n_act]), bits(out_e[l][:n_act])), f"step {step} layer {l} output"
            for which in ("k", "v"):
                a, b = bits(ga.pool_view(l, which)), bits(eb.pool_view(l, which))
                assert np.array_equal(a[:NB], b[:NB]), f"step {step} layer {l} {which} pool"
        for s in seqs:
            ctx[s] += 1
    # a step that is not pure decode is refused with nothing enqueued
    two = StepBatch(tokens=[0, 0], positions=np.array([5, 6], np.int32), query_start=np.array([0, 2], np.int32),
                    context_len=np.array([7], np.int32), block_tables=np.array(blocks[0][:1], np.int32), max_blocks=1)
    assert not ga.decode_graph(two, io)
    # a real row whose position lies past its own table is refused, as plan() refuses it (padding would
    # otherwise widen the table with the spare block and write the token there)
    bad = StepBatch(tokens=[0], positions=np.array([16], np.int32), query_start=np.array([0, 1], np.int32),
                    context_len=np.array([17], np.int32), block_tables=np.array(blocks[0][:1], np.int32), max_blocks=1)
    with pytest.raises(EmberError, match="beyond its block table"):
        ga.decode_graph(bad, io)
    with pytest.raises(EmberError, match="beyond its block table"):
        eb.plan(bad)


def test_copy_blocks_many_pairs_back_to_back(rng, device):
    """copy_blocks stages its pair lists through preallocated, double-buffered lists (no allocation, no host
    wait): 5000 pairs (more than one list holds) and then 3 more pairs right behind them, every layer, K and V,
    bit-exact."""
    NB, L = 10240, 2
    kv = PagedKv(n_layers=L, n_heads=H, n_kv_heads=KVH, max_position=256, num_blocks=NB, max_batch_tokens=64,
                 max_seqs=8, dtype=torch.float16)
    for layer in range(L):
        for which in ("k", "v"):
            pool = kv.pool_view(layer, which)
            pool.copy_(torch.randn(pool.shape, device=device).to(torch.float16))
    torch.cuda.synchronize()
    before = [[kv.pool_view(layer, which).clone() for which in ("k", "v")] for layer in range(L)]
    perm = rng.permutation(NB)
    src1, dst1 = perm[:5000], perm[5000:10000]
    src2, dst2 = perm[10000:10003], perm[10003:10006]
    kv.copy_blocks(src1, dst1)
    kv.copy_blocks(src2, dst2)
    torch.cuda.synchronize()
    for layer in range(L):
        for i, which in enumerate(("k", "v")):
            got, want = kv.pool_view(layer, which), before[layer][i].clone()
            want[torch.from_numpy(dst1).to(device)] = before[layer][i][torch.from_numpy(src1).to(device)]
            want[torch.from_numpy(dst2).to(device)] = before[layer][i][torch.from_numpy(src2).to(device)]
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"layer {layer} {which}"
    kv.close()


def test_attention_block_matches_oracle(device):
    """Two layers of the full attention block (input RMSNorm, qkv GEMV, fused append + attention, o GEMV into
    the f32 residual) on a decode step of 24 sequences, against the oracle's composition of the same pieces
    with the GPU path's f16 roundings (xn, qkv and att stored as f16, as cuda_backend.cu:350-362 does).
    Bound: the residual update within 5e-3 of the oracle's (relative to its largest element)."""
    HID = H * D
    L, NB = 2, 1024
    w = World(device, torch.float16, NB, n_layers=L, max_batch_tokens=16384, seed=5)
    rng = np.random.default_rng(21)
    S = 24
    ctx = rng.integers(20, 600, S)
    perm = rng.permutation(NB)
    mb = int((ctx.max() + PAGE) // PAGE) + 1
    tables = np.full((S, mb), -1, np.int32)
    used = 0
    for s_ in range(S):
        n = int(ctx[s_]) // PAGE + 1
        tables[s_, :n] = perm[used:used + n]
        used += n
    # a cached context first (one prefill step of random K/V through the plain path), then the block step
    qs0 = np.concatenate([[0], np.cumsum(ctx - 1)]).astype(np.int32)
    pos0 = np.concatenate([np.arange(c - 1) for c in ctx]).astype(np.int32)
    pre = _acts(rng, pos0.size, L, True)
    w.step(pos0, qs0, tables, pre, check=False)
    positions = (ctx - 1).astype(np.int32)
    qs = np.arange(S + 1, dtype=np.int32)
    T = S
    in_norm = [(1 + 0.1 * rng.standard_normal(HID)).astype(np.float32) for _ in range(L)]
    w_qkv = [(rng.standard_normal((W, HID)) * 0.03).astype(np.float16) for _ in range(L)]
    w_o = [(rng.standard_normal((HID, HID)) * 0.03).astype(np.float16) for _ in range(L)]
    h0 = rng.standard_normal((T, HID)).astype(np.float32)
    h = torch.from_numpy(h0).to(device)
    xn = torch.empty((T, HID), dtype=torch.float16, device=device)
    qkv = torch.empty((T, W), dtype=torch.float16, device=device)
    att = torch.empty((T, H, D), dtype=torch.float16, device=device)
    w.kv.plan(StepBatch(tokens=[0] * T, positions=positions.tolist(), query_start=qs.tolist(),
                        context_len=(positions + 1).tolist(), block_tables=tables.reshape(-1).tolist(), max_blocks=mb))
    for layer in range(L):
        w.kv.attention_block(layer, h, torch.from_numpy(in_norm[layer]).to(device),
                             torch.from_numpy(w_qkv[layer]).to(device), torch.from_numpy(w_o[layer]).to(device),
                             xn=xn, qkv=qkv, att=att, q_norm=w.qn_d[layer], k_norm=w.kn_d[layer])
    torch.cuda.synchronize()
    got = h.cpu().numpy()
    # the oracle: the same composition in f32 / double, rounding where the GPU path stores f16
    ho = h0.copy()
    for layer in range(L):
        xo = np.stack([oracle.rmsnorm(ho[t], in_norm[layer], EPS) for t in range(T)]).astype(np.float16)
        qkv_o = oracle.linear(xo, w_qkv[layer], 0).astype(np.float16).astype(np.float32)
        q_ref = oracle.append_layer(qkv_o, positions, qs, tables, w.ko[layer], w.vo[layer], n_heads=H, n_kv=KVH,
                                    inv_freq_=w.inv, eps=EPS, q_norm=w.qn[layer], k_norm=w.kn[layer],
                                    num_blocks=NB + 1, kv_f16=False)
        att_o = oracle.attention_layer(q_ref, positions, qs, tables, w.ko[layer], w.vo[layer], n_heads=H, n_kv=KVH,
                                       num_blocks=NB + 1, kv_f16=False, threads=8)
        ho = oracle.linear(att_o.reshape(T, HID).astype(np.float16), w_o[layer], 2, ho)
    d_got, d_want = got - h0, ho - h0
    assert np.isfinite(got).all()
    assert float(np.abs(d_got - d_want).max()) / float(np.abs(d_want).max()) < 5e-3


def test_layer_rejects_misaligned_qkv(device):
    """ember_kv_layer refuses a qkv that is not 16-byte aligned (the append kernel moves 8 elements per
    access) with an error, before any launch; the same step then runs from an aligned buffer."""
    from ember_amd import _lib

    w = World(device, torch.float16, num_blocks=8)
    w.kv.plan(StepBatch(tokens=[0], positions=[0], query_start=[0, 1], context_len=[1], block_tables=[0], max_blocks=1))
    buf = torch.zeros(W + 8, dtype=torch.float16, device=device)
    out = torch.zeros((1, H, D), dtype=torch.float16, device=device)
    rc = _lib.lib().ember_kv_layer(w.kv._h, 0, buf.data_ptr() + 2, None, None, None, out.data_ptr())
    assert rc == _lib.ERR_INVALID
    assert "16-byte aligned" in _lib.last_error()
    w.kv.layer(0, buf[:W].view(1, W), out)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()


def test_config2_full_size_decode_step(rng, device):
    """BASELINE config 2 at full size, one layer: 32 sequences with cached contexts U[256, 4096], one new token
    each, pages scattered by a random permutation of an 8192-page pool. This is the step bench.py times (fused
    append + attention, work list, in-kernel split merge): attention within 2e-3 of the oracle, and the new K/V
    slots equal to the oracle's to f16 rounding."""
    NB, S = 8192, 32
    w = World(device, torch.float16, num_blocks=NB, max_position=4096 + 2 * PAGE)
    ctx = rng.integers(256, 4097, S)
    mb = 4096 // PAGE + 2
    tables = np.zeros((S, mb), np.int32)
    pages, used = rng.permutation(NB).astype(np.int32), 0
    for s in range(S):
        n = int(ctx[s]) // PAGE + 1  # the new token at position ctx[s] included
        tables[s, :n] = pages[used:used + n]
        used += n
    # cached K/V: every slot of the pool random, the same values in the oracle's f32 pools
    for which, ref in (("k", w.ko[0]), ("v", w.vo[0])):
        pool = w.kv.pool_view(0, which)
        pool.copy_(torch.randn(pool.shape, dtype=torch.float32, device=device).mul_(0.5).to(torch.float16))
        ref[:] = pool.float().cpu().numpy()
    torch.cuda.synchronize()
    positions = ctx.astype(np.int32)
    qkv = _acts(rng, S, 1, True)
    (got, want), = w.step(positions, np.arange(S + 1, dtype=np.int32), tables, qkv)
    assert w.kv.fused(), "a pure decode step of one token per sequence runs fused"
    assert np.isfinite(got).all()
    assert rel_err(got, want) < 2e-3
    kg, vg = w.pools(0)
    for s in range(S):
        b, slot = tables[s, ctx[s] // PAGE], ctx[s] % PAGE
        np.testing.assert_allclose(kg[b, :, slot], w.ko[0][b, :, slot], rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(vg[b, :, slot], w.vo[0][b, :, slot], rtol=1e-3, atol=1e-3)


def test_config4_pool_size_and_long_contexts(rng, device):
    """BASELINE config 4's pool at one layer: 131,072 pages, so one layer's K (or V) pool is 4.3 GB and element
    offsets pass 2^31, and contexts up to 16,384 tokens (32 splits of 512). Four sequences whose pages sit at the
    top of the pool take a fused decode step through the path; the oracle gets a compacted copy of their pages."""
    NB = 131072
    kv = PagedKv(n_layers=1, n_heads=H, n_kv_heads=KVH, rms_eps=EPS, rope_theta=THETA, max_position=16384 + 2 * PAGE,
                 num_blocks=NB, max_batch_tokens=64, max_seqs=8, dtype=torch.float16)
    ctx = np.array([16384, 9000, 12345, 700])
    S, mb = len(ctx), 16384 // PAGE + 2
    top = rng.permutation(np.arange(NB - 4096, NB)).astype(np.int32)
    tables, compact, used = np.zeros((S, mb), np.int32), np.zeros((S, mb), np.int32), 0
    for s in range(S):
        n = int(ctx[s]) // PAGE + 1  # the new token's page included
        tables[s, :n], compact[s, :n] = top[used:used + n], np.arange(used, used + n)
        used += n
    ko, vo = np.zeros((used + 1, KVH, PAGE, D), np.float32), np.zeros((used + 1, KVH, PAGE, D), np.float32)
    idx = torch.from_numpy(np.concatenate([tables[s, :int(ctx[s]) // PAGE + 1] for s in range(S)]).astype(np.int64))
    for which, ref in (("k", ko), ("v", vo)):
        vals = (0.5 * torch.randn((used, KVH, PAGE, D), dtype=torch.float32)).to(torch.float16)
        kv.pool_view(0, which)[idx.to(device)] = vals.to(device)
        ref[:used] = vals.float().numpy()
    positions, qs = ctx.astype(np.int32), np.arange(S + 1, dtype=np.int32)
    qkv = rng.standard_normal((S, W)).astype(np.float16)
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kv.plan(StepBatch(tokens=[0] * S, positions=positions.tolist(), query_start=qs.tolist(),
                      context_len=(ctx + 1).tolist(), block_tables=tables.reshape(-1).tolist(), max_blocks=mb))
    out = torch.full((S, H, D), float("nan"), dtype=torch.float16, device=device)
    kv.layer(0, torch.from_numpy(qkv).to(device), out, q_norm=torch.from_numpy(qn).to(device),
             k_norm=torch.from_numpy(kn).to(device))
    torch.cuda.synchronize()
    assert kv.fused()
    q_ref = oracle.append_layer(qkv.astype(np.float32), positions, qs, compact, ko, vo, n_heads=H, n_kv=KVH,
                                inv_freq_=oracle.inv_freq(THETA, D), eps=EPS, q_norm=qn, k_norm=kn, num_blocks=used + 1,
                                kv_f16=False)
    want = oracle.attention_layer(q_ref, positions, qs, compact, ko, vo, n_heads=H, n_kv=KVH, num_blocks=used + 1,
                                  kv_f16=False, threads=8)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, want) < 2e-3
    del kv
