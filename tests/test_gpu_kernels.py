"""GPU parity of the gfx950 kernels, called through the C ABI, against the CPU oracle.

Tolerances (north star): page placement and slot indices bit-exact; attention
within 2e-3 relative error for f16 KV and 1e-5 for f32 KV, where the relative
error of a result is max|got - want| / max|want| over each (token, head)
vector, worst vector reported (helpers.rel_err).
"""
import numpy as np
import pytest
import torch

import oracle
from ember_amd import kernels as K
from helpers import D, PAGE, attention_f64, make_step, rel_err

pytestmark = pytest.mark.gpu

H, KVH = 16, 8
W = (H + 2 * KVH) * D
THETA = 1e6


def _pools(NB, dtype, fill=0.0, dev="cuda"):
    k = torch.full((NB, KVH, PAGE, D), fill, dtype=dtype, device=dev)
    return k, k.clone()


def _host(t):
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.float16 else a


def _random_pools(rng, step, NB, f16):
    """Pools holding random K/V at every cached position, NaN in every other slot (never written)."""
    k = np.full((NB, KVH, PAGE, D), np.nan, np.float32)
    v = k.copy()
    for s in range(step.S):
        ctx = int(step.positions[step.query_start[s + 1] - 1]) + 1
        for p0 in range(0, ctx, PAGE):
            b = step.tables[s, p0 // PAGE]
            n = min(PAGE, ctx - p0)
            k[b, :, :n] = rng.standard_normal((KVH, n, D)) * 0.35
            v[b, :, :n] = rng.standard_normal((KVH, n, D))
    if f16:
        k, v = k.astype(np.float16), v.astype(np.float16)
    return k, v


# ---- fused QK-norm + RoPE + append ----

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("bias,norm", [(False, True), (True, True), (False, False)])
def test_append_matches_oracle(rng, device, dtype, bias, norm):
    NB = 64
    step = make_step(rng, [1, 16, 17, 200, 33], [1, 16, 2, 5, 3], NB)
    qkv = rng.standard_normal((step.T, W)).astype(np.float32)
    qn = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32) if norm else None
    kn = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32) if norm else None
    bs = (0.1 * rng.standard_normal(W)).astype(np.float32) if bias else None
    f16 = dtype == torch.float16
    qkv_in = qkv.astype(np.float16) if f16 else qkv
    inv = oracle.inv_freq(THETA, D)
    # Sentinel pools: a slot never written keeps its NaN pattern.
    sent = np.uint16(0x7E01)
    kp, vp = _pools(NB, dtype, float("nan"), device)
    if f16:
        kp.view(torch.int16).fill_(int(sent))
        vp.view(torch.int16).fill_(int(sent))
    q_out = torch.empty((step.T, H, D), dtype=dtype, device=device)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    dv = lambda a: None if a is None else torch.from_numpy(a).to(device)  # noqa: E731
    K.qk_norm_rope_store(torch.from_numpy(qkv_in).to(device), q_out, kp, vp, ints, n_heads=H, n_kv=KVH,
                         inv_freq_dev=dv(inv), q_norm=dv(qn), k_norm=dv(kn), bias=dv(bs))
    torch.cuda.synchronize()

    ko = np.full((NB, KVH, PAGE, D), sent if f16 else np.nan, np.uint16 if f16 else np.float32)
    vo = ko.copy()
    q_ref = oracle.append_layer(qkv_in.astype(np.float32), step.positions, step.query_start, step.tables, ko, vo,
                                n_heads=H, n_kv=KVH, inv_freq_=inv, q_norm=qn, k_norm=kn, bias=bs, num_blocks=NB,
                                kv_f16=f16)
    kg, vg = _host(kp), _host(vp)
    written = (lambda a: a != sent) if f16 else (lambda a: ~np.isnan(a))
    written_o = written(ko)
    assert np.array_equal(written(kg), written_o), "the set of written K slots differs"
    assert np.array_equal(written(vg), written(vo)) and np.array_equal(written(vo), written_o)
    assert np.array_equal(vg[written_o], vo[written_o])  # V is stored as given (clamped and rounded in f16)
    if f16:
        kgf, kof = kg.view(np.float16).astype(np.float32), ko.view(np.float16).astype(np.float32)
        diff_bits = np.abs(kg.astype(np.int32) - ko.astype(np.int32))[written_o]
        assert diff_bits.max() <= 1, "K differs from the oracle by more than one f16 ulp"
        assert (diff_bits == 0).mean() > 0.999
        qg = q_out.float().cpu().numpy()
        np.testing.assert_allclose(qg, q_ref.astype(np.float16).astype(np.float32), rtol=1e-3, atol=1e-3)
        assert np.isfinite(kgf[written_o]).all() and np.isfinite(kof[written_o]).all()
    else:
        np.testing.assert_allclose(kg[written_o], ko[written_o], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(q_out.cpu().numpy(), q_ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("heads", [(12, 4), (4, 2)], ids=["12q4kv", "4q2kv"])
def test_append_waves_mixing_query_and_kv_heads(rng, device, dtype, heads):
    """A wave holds 8 heads: with 12 / 4 heads its second wave holds 4 query and 4 K heads and its third 4 V heads
    and 4 dead lanes; with 4 / 2 one wave holds query, K and V heads. Write set, V bits and K against the oracle."""
    h, kvh = heads
    NB, w = 48, (h + 2 * kvh) * D
    step = make_step(rng, [1, 40, 200], [1, 3, 17], NB)
    qkv = rng.standard_normal((step.T, w)).astype(np.float32)
    f16 = dtype == torch.float16
    qkv_in = qkv.astype(np.float16) if f16 else qkv
    qn = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    inv = oracle.inv_freq(THETA, D)
    kp = torch.full((NB, kvh, PAGE, D), float("nan"), dtype=torch.float32, device=device).to(dtype)
    vp = kp.clone()
    q_out = torch.empty((step.T, h, D), dtype=dtype, device=device)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    dv = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    K.qk_norm_rope_store(dv(qkv_in), q_out, kp, vp, ints, n_heads=h, n_kv=kvh, inv_freq_dev=dv(inv), q_norm=dv(qn),
                         k_norm=dv(kn))
    torch.cuda.synchronize()
    # The oracle's f16 pools are f16 bits, NaN-filled as the device pools are.
    ko = np.full((NB, kvh, PAGE, D), np.nan, np.float16).view(np.uint16) if f16 else \
        np.full((NB, kvh, PAGE, D), np.nan, np.float32)
    vo = ko.copy()
    q_ref = oracle.append_layer(qkv_in.astype(np.float32), step.positions, step.query_start, step.tables, ko, vo,
                                n_heads=h, n_kv=kvh, inv_freq_=inv, q_norm=qn, k_norm=kn, num_blocks=NB, kv_f16=f16)
    kg, vg = kp.float().cpu().numpy(), vp.float().cpu().numpy()
    if f16:
        ko, vo = ko.view(np.float16).astype(np.float32), vo.view(np.float16).astype(np.float32)
    written = ~np.isnan(ko)
    assert written.sum() == step.T * kvh * D
    assert np.array_equal(~np.isnan(kg), written) and np.array_equal(~np.isnan(vg), ~np.isnan(vo))
    assert np.array_equal(vg[written], vo[written])
    tol = 2e-3 if f16 else 1e-5  # f16: K within one f16 ulp of the oracle's rounding
    np.testing.assert_allclose(kg[written], ko[written], rtol=tol, atol=tol)
    np.testing.assert_allclose(q_out.float().cpu().numpy(), q_ref, rtol=tol, atol=tol)


def test_append_far_positions_and_clamp(rng, device):
    """Positions up to 40959 (Qwen3 max), and V beyond the f16 range is clamped to +-65504."""
    NB = 2700  # 2560 + 63 pages for the two contexts
    step = make_step(rng, [40960, 1000], [2, 1], NB, max_blocks=2560)
    qkv = rng.standard_normal((step.T, W)).astype(np.float32)
    qkv[:, (H + KVH) * D:(H + KVH) * D + 4] = [1e5, -1e5, 7e4, 65504.0]
    kp, vp = _pools(NB, torch.float32, 0.0, device)
    q_out = torch.empty((step.T, H, D), dtype=torch.float32, device=device)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    inv = oracle.inv_freq(THETA, D)
    K.qk_norm_rope_store(torch.from_numpy(qkv).to(device), q_out, kp, vp, ints, n_heads=H, n_kv=KVH,
                         inv_freq_dev=torch.from_numpy(inv).to(device),
                         q_norm=torch.ones(D, device=device), k_norm=torch.ones(D, device=device))
    ko, vo = np.zeros((NB, KVH, PAGE, D), np.float32), np.zeros((NB, KVH, PAGE, D), np.float32)
    q_ref = oracle.append_layer(qkv, step.positions, step.query_start, step.tables, ko, vo, n_heads=H, n_kv=KVH,
                                inv_freq_=inv, q_norm=np.ones(D, np.float32), k_norm=np.ones(D, np.float32),
                                num_blocks=NB, kv_f16=False)
    torch.cuda.synchronize()
    np.testing.assert_allclose(q_out.cpu().numpy(), q_ref, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(kp.cpu().numpy(), ko, rtol=2e-5, atol=2e-5)
    # f16 pools clamp V
    kh, vh = _pools(NB, torch.float16, 0.0, device)
    qh = torch.empty((step.T, H, D), dtype=torch.float16, device=device)
    K.qk_norm_rope_store(torch.from_numpy(qkv.astype(np.float16)).to(device), qh, kh, vh, ints, n_heads=H, n_kv=KVH,
                         inv_freq_dev=torch.from_numpy(inv).to(device),
                         q_norm=torch.ones(D, device=device), k_norm=torch.ones(D, device=device))
    torch.cuda.synchronize()
    t = step.T - 1
    s, p = step.token_seq[t], step.positions[t]
    row = vh[step.tables[s, p // PAGE], 0, p % PAGE, :4].float().cpu().numpy()
    assert row.tolist() == [65504.0, -65504.0, 65504.0, 65504.0]



def test_append_writes_nothing_for_a_slot_outside_the_table(device):
    """Through the C ABI (the Python wrapper refuses such steps), a token whose position lies past its block
    table, and one at position -1 with sequence -1, store nothing; a valid token in the same launch stores the
    same bits, and gets the same q, as when it is appended alone. The kernel looks up every token's block id
    unguarded, its index clamped into the row (row 0 for a negative sequence)."""
    import ctypes

    from ember_amd import _lib

    NB, MB = 8, 2
    rng = np.random.default_rng(11)
    tables = torch.tensor([[3, 5]], dtype=torch.int32, device=device)
    inv = torch.from_numpy(oracle.inv_freq(THETA, D)).to(device)
    ones = torch.ones(D, device=device)

    def run(positions, seqs):
        T = len(positions)
        qkv = torch.from_numpy(rng_qkv[:T]).to(device)
        q_out = torch.zeros((T, H, D), dtype=torch.float16, device=device)
        kp, vp = _pools(NB, torch.float16, 7.0, device)
        pos = torch.tensor(positions, dtype=torch.int32, device=device)
        seq = torch.tensor(seqs, dtype=torch.int32, device=device)
        a = _lib.QkvArgs()
        a.qkv, a.q_out, a.k_cache, a.v_cache = qkv.data_ptr(), q_out.data_ptr(), kp.data_ptr(), vp.data_ptr()
        a.q_norm, a.k_norm, a.bias, a.inv_freq = ones.data_ptr(), ones.data_ptr(), None, inv.data_ptr()
        a.positions, a.token_seq, a.block_tables = pos.data_ptr(), seq.data_ptr(), tables.data_ptr()
        a.max_blocks, a.T, a.n_heads, a.n_kv, a.head_dim = MB, T, H, KVH, D
        a.eps, a.num_blocks, a.dtype = 1e-6, NB, _lib.DTYPE_F16
        _lib.check(_lib.lib().ember_hip_kv_append(ctypes.byref(a), None), "kv_append")
        torch.cuda.synchronize()
        return _host(q_out), _host(kp), _host(vp)

    rng_qkv = (rng.standard_normal((3, W)) * 0.5).astype(np.float16)
    q3, k3, v3 = run([5, MB * PAGE, -1], [0, 0, -1])
    q1, k1, v1 = run([5], [0])
    sentinel = np.full((NB, KVH, PAGE, D), 7.0, np.float16).view(np.uint16)
    written = np.zeros((NB, KVH, PAGE, D), bool)
    written[3, :, 5, :] = True
    for pool3, pool1 in ((k3, k1), (v3, v1)):
        assert np.array_equal(pool3[~written], sentinel[~written])  # nothing else was written
        assert np.array_equal(pool3, pool1)                         # the valid token's slot, same bits
        assert not np.array_equal(pool3[written], sentinel[written])
    assert np.array_equal(q3[0], q1[0])


# ---- paged decode attention ----

def _run_decode(q, kp, vp, step, NB, device, **kw):
    dtype = kp.dtype
    out = torch.full((step.T, H, D), float("nan"), dtype=dtype, device=device)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    K.paged_attention(torch.from_numpy(q).to(device), kp, vp, out, ints, n_heads=H, n_kv=KVH, **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("split_len,work", [(16, False), (64, True), (512, False), (512, True), (512, "pairs"),
                                            (1024, False), (1024, True)])
def test_decode_f32_matches_oracle(rng, device, split_len, work):
    """work: False = dense grid; True = sorted work list with the plan's per-item descriptors; "pairs" = the
    work list alone (the kernel looks each item up)."""
    NB = 1200
    ctxs = [1, 15, 16, 17, 100, 511, 512, 513, 1500, 4096]
    step = make_step(rng, ctxs, [1] * len(ctxs), NB)
    k, v = _random_pools(rng, step, NB, f16=False)
    q = rng.standard_normal((step.T, H, D)).astype(np.float32)
    out = _run_decode(q, torch.from_numpy(k).to(device), torch.from_numpy(v).to(device), step, NB, device,
                      split_len=split_len, use_work_list=bool(work), work_desc=work is True).cpu().numpy()
    want = oracle.attention_layer(q, step.positions, step.query_start, step.tables, np.nan_to_num(k), np.nan_to_num(v),
                                  n_heads=H, n_kv=KVH, num_blocks=NB, kv_f16=False, threads=8)
    assert np.isfinite(out).all()
    assert rel_err(out, want) < 1e-5
    assert rel_err(out, attention_f64(q, step, np.nan_to_num(k), np.nan_to_num(v), H, KVH)) < 1e-5


def test_decode_f16_matches_oracle(rng, device):
    NB = 2400
    ctxs = list(rng.integers(256, 4097, 12)) + [1, 2, 16, 17]
    step = make_step(rng, ctxs, [1] * len(ctxs), NB)
    k, v = _random_pools(rng, step, NB, f16=True)
    q32 = rng.standard_normal((step.T, H, D)).astype(np.float32)
    q16 = q32.astype(np.float16)
    out = _run_decode(q16, torch.from_numpy(k).to(device), torch.from_numpy(v).to(device), step, NB, device)
    got = out.float().cpu().numpy()
    kf, vf = np.nan_to_num(k.astype(np.float32)), np.nan_to_num(v.astype(np.float32))
    # against the f32 CPU path on the same (f16-valued) inputs
    want = oracle.attention_layer(q16.astype(np.float32), step.positions, step.query_start, step.tables, kf, vf,
                                  n_heads=H, n_kv=KVH, num_blocks=NB, kv_f16=False, threads=8)
    assert rel_err(got, want) < 2e-3
    # and against the f32 CPU path with an f32 query: the error budget of f16 storage
    want32 = oracle.attention_layer(q32, step.positions, step.query_start, step.tables, kf, vf, n_heads=H, n_kv=KVH,
                                    num_blocks=NB, kv_f16=False, threads=8)
    assert rel_err(got, want32) < 2e-3


def test_decode_is_batch_invariant(rng, device):
    """A token's output is bit-identical alone, in a batch, and with any number of splits launched."""
    NB = 1600
    ctxs = [3000, 700, 64, 1, 2049]
    step = make_step(rng, ctxs, [1] * len(ctxs), NB)
    k, v = _random_pools(rng, step, NB, f16=True)
    kp, vp = torch.from_numpy(k).to(device), torch.from_numpy(v).to(device)
    q = rng.standard_normal((step.T, H, D)).astype(np.float16)
    full = _run_decode(q, kp, vp, step, NB, device).cpu().numpy().view(np.uint16)
    for t in range(step.T):
        s = step.token_seq[t]
        one = make_step(rng, [ctxs[s]], [1], NB)
        one.tables = step.tables[s:s + 1]
        alone = _run_decode(q[t:t + 1], kp, vp, one, NB, device).cpu().numpy().view(np.uint16)
        assert np.array_equal(alone[0], full[t]), f"token {t} differs alone vs in the batch"
        # a launch with more splits than this token needs (as in a batch with a longer context)
        wide = _run_decode(q[t:t + 1], kp, vp, one, NB, device, num_splits=8).cpu().numpy().view(np.uint16)
        assert np.array_equal(wide[0], full[t])


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_verify_run_equals_sequential_decode(rng, device, dtype):
    """q_len = 5 runs (speculative verify) read each page once for 5 tokens; every token's output is
    bit-identical to decoding it alone."""
    NB = 900
    base = [511, 512, 1000, 2045, 5, 16, 27]
    n = 5
    step = make_step(rng, [c + n for c in base], [n] * len(base), NB)
    f16 = dtype == torch.float16
    k, v = _random_pools(rng, step, NB, f16=f16)
    kp, vp = torch.from_numpy(k).to(device), torch.from_numpy(v).to(device)
    q = rng.standard_normal((step.T, H, D)).astype(np.float16 if f16 else np.float32)
    runs = K.decode_runs(K.StepInts(step.positions, step.token_seq, step.tables, NB), range(step.T), max_run=n)
    assert runs[1].tolist() == [n] * len(base)
    verify = _run_decode(q, kp, vp, step, NB, device, runs=runs).cpu().numpy()
    seq = _run_decode(q, kp, vp, step, NB, device).cpu().numpy()  # one run per token
    assert np.array_equal(verify.view(np.uint8), seq.view(np.uint8))
    listed = _run_decode(q, kp, vp, step, NB, device, runs=runs, use_work_list=True).cpu().numpy()
    assert np.array_equal(listed.view(np.uint8), seq.view(np.uint8))
    # runs whose entries count down: the descriptors cannot give tokens and positions arithmetically, so the
    # kernel looks each one up
    tl = np.concatenate([np.arange(a, b)[::-1] for a, b in zip(step.query_start[:-1], step.query_start[1:])])
    down = (np.arange(0, step.T, n, dtype=np.int32), np.full(len(base), n, np.int32))
    listed = _run_decode(q, kp, vp, step, NB, device, token_list=tl, runs=down, use_work_list=True).cpu().numpy()
    assert np.array_equal(listed.view(np.uint8), seq.view(np.uint8))
    # the split merge in the last work-group of each (run, kv head)
    listed = _run_decode(q, kp, vp, step, NB, device, runs=runs, use_work_list=True, merge_in_kernel=True).cpu().numpy()
    assert np.array_equal(listed.view(np.uint8), seq.view(np.uint8))
    # runs of 2 and 3 too
    for m in (2, 3, 8):
        r = K.decode_runs(K.StepInts(step.positions, step.token_seq, step.tables, NB), range(step.T), max_run=m)
        other = _run_decode(q, kp, vp, step, NB, device, runs=r).cpu().numpy()
        assert np.array_equal(other.view(np.uint8), seq.view(np.uint8))
    want = oracle.attention_layer(q.astype(np.float32), step.positions, step.query_start, step.tables,
                                  np.nan_to_num(k.astype(np.float32)), np.nan_to_num(v.astype(np.float32)),
                                  n_heads=H, n_kv=KVH, num_blocks=NB, kv_f16=False, threads=8)
    assert rel_err(verify.astype(np.float32), want) < (2e-3 if f16 else 1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_decode_group_sizes(rng, device, dtype):
    """GQA groups 1, 2, 4, 8 (n_heads / n_kv): f32 pages on the VALU, f16 pages on MFMA, where a work-group's
    G rows fill 1, 2, 4 or 8 of the 16 query columns."""
    NB = 300
    f16 = dtype == torch.float16
    nt = np.float16 if f16 else np.float32
    for g, kvh in ((1, 8), (2, 8), (4, 4), (8, 2)):
        h = g * kvh
        step = make_step(rng, [700, 33, 1], [1, 1, 1], NB)
        k = rng.standard_normal((NB, kvh, PAGE, D)).astype(nt)
        v = rng.standard_normal((NB, kvh, PAGE, D)).astype(nt)
        q = rng.standard_normal((step.T, h, D)).astype(nt)
        out = torch.empty((step.T, h, D), dtype=dtype, device=device)
        ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
        K.paged_attention(torch.from_numpy(q).to(device), torch.from_numpy(k).to(device), torch.from_numpy(v).to(device),
                          out, ints, n_heads=h, n_kv=kvh, split_len=256)
        torch.cuda.synchronize()
        want = oracle.attention_layer(q.astype(np.float32), step.positions, step.query_start, step.tables,
                                      k.astype(np.float32), v.astype(np.float32), n_heads=h, n_kv=kvh,
                                      num_blocks=NB, kv_f16=False)
        assert rel_err(out.float().cpu().numpy(), want) < (2e-3 if f16 else 1e-5), f"group {g}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_decode_out_of_pool_block_reads_as_zeros(rng, device, dtype):
    """A table entry outside the pool reads as a page of zeros (its loads are bounds-checked and touch no
    memory; EmberAttnArgs::num_blocks): equal, within tolerance, to the oracle with that entry pointing at an
    all-zero block appended to the pool. Pages in the middle of a context, on the fast path, and the last page
    (masked) are both covered, with a dense grid and with the work list and in-kernel merge."""
    NB = 400
    f16 = dtype == torch.float16
    ctxs = [900, 300, 40]
    step = make_step(rng, ctxs, [1] * len(ctxs), NB)
    k, v = _random_pools(rng, step, NB, f16=f16)
    bad = step.tables.copy()
    bad[0, 5] = NB + 7            # a middle page of sequence 0 (fast path)
    bad[1, 300 // PAGE] = NB      # the last page of sequence 1 (masked)
    zk = np.concatenate([np.nan_to_num(k.astype(np.float32)), np.zeros((1, KVH, PAGE, D), np.float32)])
    zv = np.concatenate([np.nan_to_num(v.astype(np.float32)), np.zeros((1, KVH, PAGE, D), np.float32)])
    zt = bad.copy()
    zt[0, 5] = NB
    zt[1, 300 // PAGE] = NB
    q = rng.standard_normal((step.T, H, D)).astype(np.float16 if f16 else np.float32)
    want = oracle.attention_layer(q.astype(np.float32), step.positions, step.query_start, zt, zk, zv,
                                  n_heads=H, n_kv=KVH, num_blocks=NB + 1, kv_f16=False, threads=8)
    kp, vp = torch.from_numpy(k).to(device), torch.from_numpy(v).to(device)
    for kw in ({}, {"use_work_list": True, "merge_in_kernel": True}):
        # The Python wrapper rejects such a table on the host; a C-ABI caller need not, so the table is swapped
        # in after that check. The kernel is told the true pool size (num_blocks = NB) and bounds-checks it.
        ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
        ints.block_tables = np.ascontiguousarray(bad)
        out = torch.full((step.T, H, D), float("nan"), dtype=dtype, device=device)
        keep = K.paged_attention(torch.from_numpy(q).to(device), kp, vp, out, ints, n_heads=H, n_kv=KVH, **kw)
        torch.cuda.synchronize()
        del keep
        got = out.float().cpu().numpy()
        assert np.isfinite(got).all()
        assert rel_err(got, want) < (2e-3 if f16 else 1e-5), kw


def test_copy_pages(rng, device):
    NB, L = 40, 3
    stride = NB * KVH * PAGE * D
    kp = torch.from_numpy(rng.standard_normal(L * stride).astype(np.float16)).to(device)
    vp = torch.from_numpy(rng.standard_normal(L * stride).astype(np.float16)).to(device)
    k0, v0 = kp.cpu().numpy().reshape(L, NB, -1), vp.cpu().numpy().reshape(L, NB, -1)
    src, dst = [3, 7, 11], [30, 31, 5]
    K.copy_pages(kp, vp, src, dst, n_layers=L, layer_stride=stride, n_kv=KVH, num_blocks=NB)
    torch.cuda.synchronize()
    k1, v1 = kp.cpu().numpy().reshape(L, NB, -1), vp.cpu().numpy().reshape(L, NB, -1)
    ek, ev = k0.copy(), v0.copy()
    for s, d in zip(src, dst):
        ek[:, d], ev[:, d] = k0[:, s], v0[:, s]
    assert np.array_equal(k1.view(np.uint16), ek.view(np.uint16)) and np.array_equal(v1.view(np.uint16), ev.view(np.uint16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("work,merge", [(False, False), (True, True), (False, True)])
def test_fused_decode_step_equals_append_then_decode(rng, device, dtype, work, merge):
    """ember_hip_decode_step (append + attention in one launch) leaves the same pools and outputs, to the
    bit, as ember_hip_kv_append followed by ember_hip_paged_decode; with the split merge in a second launch or
    in the last work-group of each (run, kv head)."""
    f16 = dtype == torch.float16
    NB = 1200
    cached = [0, 15, 16, 511, 512, 1000, 2049, 3, 700]
    new = [1, 1, 5, 1, 5, 1, 4, 5, 1]
    step = make_step(rng, [c + n for c, n in zip(cached, new)], new, NB)
    k, v = _random_pools(rng, step, NB, f16=f16)
    for s, (c0, n) in enumerate(zip(cached, new)):  # new slots hold stale garbage before the step
        for p_ in range(c0, c0 + n):
            k[step.tables[s, p_ // PAGE], :, p_ % PAGE] = 7.0
            v[step.tables[s, p_ // PAGE], :, p_ % PAGE] = -3.0
    qkv = rng.standard_normal((step.T, W)).astype(np.float16 if f16 else np.float32)
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    inv = torch.from_numpy(oracle.inv_freq(THETA, D)).to(device)
    dv = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    runs = (step.query_start[:-1], np.diff(step.query_start))
    # unfused
    ka, va = dv(k), dv(v)
    q_out = torch.empty((step.T, H, D), dtype=dtype, device=device)
    out_a = torch.full((step.T, H, D), float("nan"), dtype=dtype, device=device)
    K.qk_norm_rope_store(dv(qkv), q_out, ka, va, ints, n_heads=H, n_kv=KVH, inv_freq_dev=inv, q_norm=dv(qn), k_norm=dv(kn))
    K.paged_attention(q_out, ka, va, out_a, ints, n_heads=H, n_kv=KVH, runs=runs, use_work_list=work, merge_in_kernel=merge)
    # fused
    kb, vb = dv(k), dv(v)
    out_b = torch.full((step.T, H, D), float("nan"), dtype=dtype, device=device)
    K.decode_step(dv(qkv), kb, vb, out_b, ints, n_heads=H, n_kv=KVH, inv_freq_dev=inv, q_norm=dv(qn), k_norm=dv(kn),
                  runs=runs, use_work_list=work, merge_in_kernel=merge)
    torch.cuda.synchronize()
    bits = lambda t: t.cpu().numpy().view(np.uint16 if f16 else np.uint32)  # noqa: E731
    assert np.array_equal(bits(ka), bits(kb)) and np.array_equal(bits(va), bits(vb)), "pools differ"
    assert np.array_equal(bits(out_a), bits(out_b)), "attention differs"
    # and both against the oracle
    ko, vo = np.nan_to_num(k.astype(np.float32)), np.nan_to_num(v.astype(np.float32))
    q_ref = oracle.append_layer(qkv.astype(np.float32), step.positions, step.query_start, step.tables, ko, vo, n_heads=H,
                                n_kv=KVH, inv_freq_=oracle.inv_freq(THETA, D), q_norm=qn, k_norm=kn, num_blocks=NB,
                                kv_f16=False)
    want = oracle.attention_layer(q_ref, step.positions, step.query_start, step.tables, ko, vo, n_heads=H, n_kv=KVH,
                                  num_blocks=NB, kv_f16=False, threads=8)
    assert rel_err(out_b.float().cpu().numpy(), want) < (2e-3 if f16 else 1e-5)


def test_in_kernel_merge_leaves_counters_zero_and_matches(rng, device):
    """The last-arriving work-group merges; counters come back to zero for the next launch, and repeated
    launches on the same counters give the same bits as the two-launch form."""
    NB = 1500
    ctxs = [4096, 3000, 513, 512, 100, 1]
    step = make_step(rng, ctxs, [1] * len(ctxs), NB)
    k, v = _random_pools(rng, step, NB, f16=True)
    kp, vp = torch.from_numpy(k).to(device), torch.from_numpy(v).to(device)
    q = rng.standard_normal((step.T, H, D)).astype(np.float16)
    two = _run_decode(q, kp, vp, step, NB, device, use_work_list=True).cpu().numpy().view(np.uint16)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    qd = torch.from_numpy(q).to(device)
    a, keep = K._attn_args(qd, kp, vp, torch.empty((step.T, H, D), dtype=torch.float16, device=device), ints,
                           n_heads=H, n_kv=KVH, token_list=None, runs=None, split_len=512, num_splits=None, scratch=None,
                           use_work_list=True, merge_in_kernel=True)
    out = torch.empty((step.T, H, D), dtype=torch.float16, device=device)
    a.out = out.data_ptr()
    from ember_amd import _lib
    for _ in range(3):
        out.fill_(float("nan"))
        _lib.check(_lib.lib().ember_hip_paged_decode(a, torch.cuda.current_stream().cuda_stream), "paged_decode")
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), two)
        assert int(keep[-1].abs().sum()) == 0, "merge counters not reset"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_in_kernel_merge_of_runs_across_a_split_boundary(rng, device, dtype):
    """Runs of 5 tokens whose positions straddle a split boundary (their rows merge 1 or 2 splits, 8 or 9):
    the in-kernel merge equals the merge kernel to the bit, launch after launch on the same buffers, and
    leaves the counters zero."""
    f16 = dtype == torch.float16
    NB = 1500
    cached = [508, 1021, 4094, 3, 512]
    new = [5, 5, 5, 5, 5]
    step = make_step(rng, [c + n for c, n in zip(cached, new)], new, NB)
    k, v = _random_pools(rng, step, NB, f16=f16)
    kp, vp = torch.from_numpy(k).to(device), torch.from_numpy(v).to(device)
    q = rng.standard_normal((step.T, H, D)).astype(np.float16 if f16 else np.float32)
    runs = (step.query_start[:-1], np.diff(step.query_start))
    bits = lambda t: t.cpu().numpy().view(np.uint16 if f16 else np.uint32)  # noqa: E731
    want = bits(_run_decode(q, kp, vp, step, NB, device, runs=runs, use_work_list=True, merge_in_kernel=False))
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    out = torch.empty((step.T, H, D), dtype=dtype, device=device)
    qd = torch.from_numpy(q).to(device)  # alive for every launch below: the arguments hold only its address
    a, keep = K._attn_args(qd, kp, vp, out, ints, n_heads=H, n_kv=KVH, token_list=None, runs=runs, split_len=512,
                           num_splits=None, scratch=None, use_work_list=True, merge_in_kernel=True)
    from ember_amd import _lib
    for _ in range(3):
        out.fill_(float("nan"))
        _lib.check(_lib.lib().ember_hip_paged_decode(a, torch.cuda.current_stream().cuda_stream), "paged_decode")
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), want)
        assert int(keep[-1].abs().sum()) == 0, "merge counters not reset"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("new", [1, 5])
def test_in_kernel_merge_of_many_splits(rng, device, dtype, new):
    """Runs holding from 1 to 1,032 splits: one chunk, one batch or several batches of the in-kernel merge's
    loads, and for the longest contexts at 16 keys a split more than its LDS stages (the element-by-element
    merge). Bit for bit the
    merge kernel's output, and at 512 keys a split within tolerance of the oracle up to 5k keys. (The
    16.5k-key run, summed in f32 from 33 partials, is checked bit for bit against the merge kernel only: at 64
    keys a split, from 258 partials, it lay 1.1e-5 from the oracle's single pass.)"""
    f16 = dtype == torch.float16
    NB = 2400
    cached = [16500, 5000, 4100, 1100, 300, 20]
    step = make_step(rng, [c + new for c in cached], [new] * len(cached), NB)
    k, v = _random_pools(rng, step, NB, f16=f16)
    kp, vp = torch.from_numpy(k).to(device), torch.from_numpy(v).to(device)
    q = rng.standard_normal((step.T, H, D)).astype(np.float16 if f16 else np.float32)
    runs = (step.query_start[:-1], np.diff(step.query_start)) if new > 1 else None
    bits = lambda t: t.cpu().numpy().view(np.uint16 if f16 else np.uint32)  # noqa: E731
    for split_len in (16, 64, 512):
        kw = dict(runs=runs, split_len=split_len, use_work_list=True)
        want = _run_decode(q, kp, vp, step, NB, device, merge_in_kernel=False, **kw)
        for _ in range(2):
            got = _run_decode(q, kp, vp, step, NB, device, merge_in_kernel=True, **kw)
            assert np.array_equal(bits(got), bits(want)), split_len
    ref = oracle.attention_layer(q, step.positions, step.query_start, step.tables, np.nan_to_num(k), np.nan_to_num(v),
                                 n_heads=H, n_kv=KVH, num_blocks=NB, kv_f16=f16, threads=8)
    rows = slice(int(step.query_start[1]), None)  # every run but the 16.5k-key one
    assert rel_err(want.float().cpu().numpy()[rows], ref[rows]) < (2e-3 if f16 else 1e-5)


# ---- MFMA prefill tiles ----

def _tiles_of(step, tile=64):
    """Each sequence's new tokens cut into tiles of up to `tile` consecutive tokens."""
    out = []
    for s in range(step.S):
        for a in range(int(step.query_start[s]), int(step.query_start[s + 1]), tile):
            out.append((a, min(a + tile, int(step.query_start[s + 1])), s))
    return out


@pytest.mark.parametrize("n_kv", [8, 16, 4])
def test_prefill_matches_oracle(rng, device, n_kv):
    """Chunked-prefill tiles on MFMA (causal within the chunk, over cached context before it) against the
    f32 CPU path on the same f16 inputs and a float64 textbook reference: within 2e-3. G = 2, 1, 4."""
    NB = 1500
    ctxs = [16, 64, 65, 100, 700, 1040, 2000, 17]
    new = [16, 64, 65, 100, 128, 16, 64, 17]  # the chunk: positions ctx - new .. ctx - 1
    step = make_step(rng, ctxs, new, NB)
    k = np.full((NB, n_kv, PAGE, D), np.nan, np.float32)
    v = k.copy()
    for s, c in enumerate(ctxs):
        for p0 in range(0, c, PAGE):
            n = min(PAGE, c - p0)
            k[step.tables[s, p0 // PAGE], :, :n] = rng.standard_normal((n_kv, n, D)) * 0.35
            v[step.tables[s, p0 // PAGE], :, :n] = rng.standard_normal((n_kv, n, D))
    k16, v16 = k.astype(np.float16), v.astype(np.float16)
    q16 = rng.standard_normal((step.T, H, D)).astype(np.float16)
    out = torch.full((step.T, H, D), float("nan"), dtype=torch.float16, device=device)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    K.prefill_attention(torch.from_numpy(q16).to(device), torch.from_numpy(k16).to(device),
                        torch.from_numpy(v16).to(device), out, ints, n_heads=H, n_kv=n_kv, tiles=_tiles_of(step))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    kf, vf = np.nan_to_num(k16.astype(np.float32)), np.nan_to_num(v16.astype(np.float32))
    want = oracle.attention_layer(q16.astype(np.float32), step.positions, step.query_start, step.tables, kf, vf,
                                  n_heads=H, n_kv=n_kv, num_blocks=NB, kv_f16=False, threads=8)
    assert rel_err(got, want) < 2e-3
    assert rel_err(got, attention_f64(q16.astype(np.float32), step, kf, vf, H, n_kv)) < 2e-3


def test_prefill_tile_is_independent_of_its_neighbours(rng, device):
    """A tile's output is bit-identical launched alone or with other tiles, and tokens past a tile's end
    are not written."""
    NB = 400
    step = make_step(rng, [300, 130], [100, 70], NB)
    k, v = _random_pools(rng, step, NB, f16=True)
    kp, vp = torch.from_numpy(np.nan_to_num(k)).to(device), torch.from_numpy(np.nan_to_num(v)).to(device)
    q = torch.from_numpy(rng.standard_normal((step.T, H, D)).astype(np.float16)).to(device)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    tiles = _tiles_of(step)
    both = torch.full((step.T, H, D), float("nan"), dtype=torch.float16, device=device)
    K.prefill_attention(q, kp, vp, both, ints, n_heads=H, n_kv=KVH, tiles=tiles)
    for t in tiles:
        one = torch.full((step.T, H, D), float("nan"), dtype=torch.float16, device=device)
        K.prefill_attention(q, kp, vp, one, ints, n_heads=H, n_kv=KVH, tiles=[t])
        torch.cuda.synchronize()
        a, b = one.cpu().numpy().view(np.uint16), both.cpu().numpy().view(np.uint16)
        assert np.array_equal(a[t[0]:t[1]], b[t[0]:t[1]])
        rest = np.ones(step.T, bool)
        rest[t[0]:t[1]] = False
        assert np.isnan(one.float().cpu().numpy()[rest]).all(), "a tile wrote outside its tokens"


@pytest.mark.parametrize("n_kv", [8, 4])
def test_prefill_heads_per_group_gives_the_same_bits(rng, device, n_kv):
    """One query head per work-group (heads_per_group 1) or two (2, the default at even G): every row's output
    is the same bits, so a planner may pick per launch. Tiles of several lengths, some over long context."""
    NB = 800
    ctxs, new = [64, 200, 1100, 2100, 40], [64, 120, 100, 64, 40]
    step = make_step(rng, ctxs, new, NB)
    k, v = _random_pools(rng, step, NB, f16=True)
    kp, vp = torch.from_numpy(np.nan_to_num(k)).to(device), torch.from_numpy(np.nan_to_num(v)).to(device)
    q = torch.from_numpy(rng.standard_normal((step.T, H, D)).astype(np.float16)).to(device)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    outs = []
    for hg in (0, 1, 2):
        o = torch.full((step.T, H, D), float("nan"), dtype=torch.float16, device=device)
        K.prefill_attention(q, kp, vp, o, ints, n_heads=H, n_kv=n_kv, tiles=_tiles_of(step), heads_per_group=hg)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0].float()).all()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(outs[0].view(torch.int16), outs[2].view(torch.int16))


# ---- the layer either side: decode-sized linear layers and the input RMSNorm ----

def _linear_err(got, want):
    """The reference's GEMM test metric (tests/test_cuda.cpp:49-54): max |got - want| / max(1e-3, max |want|)."""
    return float(np.abs(got.astype(np.float64) - want).max() / max(1e-3, float(np.abs(want).max())))


@pytest.mark.parametrize("M,N,KD", [(1, 256, 512), (3, 130, 256), (8, 512, 1024), (13, 200, 128), (31, 384, 512),
                                   (64, 256, 1024), (32, 4096, 2048), (32, 2048, 2048), (17, 48, 32),
                                   (16, 1024, 2048), (8, 1024, 3072), (5, 4096, 1024),
                                   (8, 2048, 6144), (16, 1024, 12288),
                                   (3, 70000, 256), (16, 66000, 1024)])
@pytest.mark.parametrize("ep", [0, 1, 2, 3])
@pytest.mark.parametrize("split", [False, True])
def test_gemv_matches_oracle(device, M, N, KD, ep, split):
    """Every epilogue on the reference test's decode-sized shapes (K a multiple of 32) and the Qwen3 projections;
    ragged M and N exercise the clamped rows. With a workspace, the shapes with few features and K beyond 4096
    take the K split: 8 x 2048 x 6144 in 2 slices and 16 x 1024 x 12288 in 4, each slice 12 k steps per wave (a
    round of 8, then one of 4). Unsplit, 16 x 1024 x 2048 and 8 x 1024 x 3072 run 8 and 12 steps per wave, 5 x
    4096 x 1024 4, and the short shapes 1 to 3. 70,000 and 66,000 features take the wide form (four tiles per
    work-group; the last block ragged). Bound 2e-3 as in the reference's test."""
    from ember_amd import _lib
    rng = np.random.default_rng(M * 7919 + N * 31 + KD + ep)
    a = (rng.standard_normal((M, KD))).astype(np.float16)
    w = (rng.standard_normal((N, KD)) * 0.05).astype(np.float16)
    cols = N // 2 if ep == _lib.EPILOGUE_SILU_MUL else N
    f32 = ep in (_lib.EPILOGUE_STORE_F32, _lib.EPILOGUE_ADD_F32)
    c0 = np.ones((M, cols), np.float32)
    c = torch.from_numpy(c0).to(device) if f32 else torch.full((M, cols), float("nan"), dtype=torch.float16,
                                                                 device=device)
    ws = K.gemv_workspace(M, N, KD, device) if split else None
    K.gemv(torch.from_numpy(a).to(device), torch.from_numpy(w).to(device), c, ep, workspace=ws)
    torch.cuda.synchronize()
    got = c.float().cpu().numpy()
    want = oracle.linear(a, w, ep, c0 if ep == _lib.EPILOGUE_ADD_F32 else None)
    assert np.isfinite(got).all()
    assert _linear_err(got, want) < 2e-3


@pytest.mark.parametrize("N,KD", [(4096, 2048), (2048, 2048), (2048, 6144), (1024, 3072)])
@pytest.mark.parametrize("ep", [0, 2])
def test_gemv_rows_do_not_depend_on_the_batch(device, N, KD, ep):
    """A token's outputs are the same bits whatever the batch around it. The batches here take both activation
    paths: up to 32 rows of a 2048-wide K slice (16 of a 3072-wide one) are staged in LDS, more rows are read
    straight from A. With fewer than 256 feature blocks (2048 and 1024 features) a batch of more than 16 tokens
    runs one 16-token tile per work-group. The split shape (2048 x 6144 over 2 slices) goes through the merge."""
    from ember_amd import _lib
    rng = np.random.default_rng(N + KD + ep)
    a = torch.from_numpy(rng.standard_normal((64, KD)).astype(np.float16)).to(device)
    w = torch.from_numpy((rng.standard_normal((N, KD)) * 0.05).astype(np.float16)).to(device)
    start = torch.from_numpy(rng.standard_normal((64, N)).astype(np.float32)).to(device)
    ws = K.gemv_workspace(64, N, KD, device)
    outs = {}
    for M in (64, 48, 32, 9, 1):
        c = start[:M].clone() if ep == _lib.EPILOGUE_ADD_F32 else torch.empty((M, N), dtype=torch.float16,
                                                                              device=device)
        K.gemv(a[:M].contiguous(), w, c, ep, workspace=ws)
        outs[M] = c
    torch.cuda.synchronize()
    view = torch.int32 if ep == _lib.EPILOGUE_ADD_F32 else torch.int16
    for M in (48, 32, 9, 1):
        assert torch.equal(outs[64][:M].view(view), outs[M].view(view)), f"M={M}"
    want = oracle.linear(a.cpu().numpy(), w.cpu().numpy(), ep,
                         start.cpu().numpy() if ep == _lib.EPILOGUE_ADD_F32 else None)
    assert _linear_err(outs[64].float().cpu().numpy(), want) < 2e-3


def test_gemv_split_is_deterministic_and_leaves_counters_zero(device):
    """The K-split merge: Qwen3-1.7B's down projection shape (2048 features, K 6144 in 2 slices) gives the same
    bits on every launch (the slices are added in slice order, whichever work-group merges), agrees with the
    unsplit launch within f32 reassociation, leaves its counters at zero, and a smaller batch right after reuses
    the workspace."""
    from ember_amd import _lib
    rng = np.random.default_rng(5)
    M, N, KD = 32, 2048, 6144
    a = torch.from_numpy(rng.standard_normal((M, KD)).astype(np.float16)).to(device)
    w = torch.from_numpy((rng.standard_normal((N, KD)) * 0.05).astype(np.float16)).to(device)
    ws = K.gemv_workspace(M, N, KD, device)
    assert ws is not None
    outs = []
    for _ in range(3):
        c = torch.zeros((M, N), dtype=torch.float32, device=device)
        K.gemv(a, w, c, _lib.EPILOGUE_ADD_F32, workspace=ws)
        outs.append(c.cpu().numpy())
    torch.cuda.synchronize()
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    plain = torch.zeros((M, N), dtype=torch.float32, device=device)
    K.gemv(a, w, plain, _lib.EPILOGUE_ADD_F32)
    np.testing.assert_allclose(outs[0], plain.cpu().numpy(), rtol=1e-5, atol=1e-4)
    assert not ws[: (N // 16) * 4].any(), "a merge counter was left non-zero"
    want = oracle.linear(a.cpu().numpy(), w.cpu().numpy(), _lib.EPILOGUE_STORE_F16, None)
    small = torch.full((5, N), float("nan"), dtype=torch.float16, device=device)
    K.gemv(a[:5].contiguous(), w, small, _lib.EPILOGUE_STORE_F16, workspace=ws)
    torch.cuda.synchronize()
    assert _linear_err(small.float().cpu().numpy(), want[:5]) < 2e-3
    assert not ws[: (N // 16) * 4].any()


def _pack_reference(w):
    """The packed layout by its definition: tile t, k step s, lane l = 16 g + c holds w[16 t + c, 32 s + 8 g: +8]."""
    N, K = w.shape
    T = (N + 15) // 16
    wp = np.zeros((T * 16, K), w.dtype)
    wp[:N] = w
    return wp.reshape(T, 16, K // 32, 4, 8).transpose(0, 2, 3, 1, 4).reshape(-1)


def test_gemv_pack_layout(device):
    rng = np.random.default_rng(8)
    for N, KD in [(16, 32), (37, 64), (4096, 1024)]:
        w = (rng.standard_normal((N, KD))).astype(np.float16)
        got = K.gemv_pack(torch.from_numpy(w).to(device)).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint16), _pack_reference(w).view(np.uint16))


@pytest.mark.parametrize("M,N,KD", [(1, 256, 512), (3, 130, 256), (16, 1024, 2048), (32, 4096, 2048),
                                   (8, 1024, 3072), (8, 2048, 6144), (64, 256, 1024), (3, 70000, 256), (17, 48, 32)])
@pytest.mark.parametrize("ep", [0, 1, 2, 3])
def test_gemv_packed_equals_row_major(device, M, N, KD, ep):
    """A packed W changes only where each lane's 16 bytes come from: the product is the same bits, with and without
    the K split, in the wide form, and with a ragged last tile (rows past N are zero in the packed copy)."""
    from ember_amd import _lib
    rng = np.random.default_rng(M * 17 + N + KD + ep)
    a = torch.from_numpy(rng.standard_normal((M, KD)).astype(np.float16)).to(device)
    w = torch.from_numpy((rng.standard_normal((N, KD)) * 0.05).astype(np.float16)).to(device)
    wp = K.gemv_pack(w)
    cols = N // 2 if ep == _lib.EPILOGUE_SILU_MUL else N
    f32 = ep in (_lib.EPILOGUE_STORE_F32, _lib.EPILOGUE_ADD_F32)
    start = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float32)).to(device)
    for split in (False, True):
        ws = K.gemv_workspace(M, N, KD, device) if split else None
        outs = []
        for packed in (None, wp):
            c = start.clone() if f32 else torch.full((M, cols), float("nan"), dtype=torch.float16, device=device)
            K.gemv(a, w, c, ep, workspace=ws, packed=packed)
            outs.append(c)
        torch.cuda.synchronize()
        view = torch.int32 if f32 else torch.int16
        assert torch.equal(outs[0].view(view), outs[1].view(view)), f"split={split}"


def test_gemv_saturates_f16_outputs(device):
    """store_f16 clamps to the finite f16 range instead of overflowing to inf (k_gemm.cu's to_half_sat)."""
    a = np.full((2, 64), 100.0, np.float16)
    w = np.full((16, 64), 50.0, np.float16)
    w[1::2] *= -1
    c = torch.empty((2, 16), dtype=torch.float16, device=device)
    K.gemv(torch.from_numpy(a).to(device), torch.from_numpy(w).to(device), c, 0)
    torch.cuda.synchronize()
    assert c.float().cpu().numpy()[0, :2].tolist() == [65504.0, -65504.0]


@pytest.mark.parametrize("ep", [0, 1, 2, 3])
def test_gemv_vector_and_scalar_stores_agree(device, ep):
    """A 16-byte aligned output whose row length is a multiple of 4 takes each lane's outputs in one store (and,
    adding into f32, one load); 130 features (rows of 130, or 65 after the SiLU pairs) take them one at a time.
    The first 128 features (64 SiLU outputs) are the same bits either way."""
    from ember_amd import _lib
    rng = np.random.default_rng(130 + ep)
    silu = ep == _lib.EPILOGUE_SILU_MUL
    a = torch.from_numpy(rng.standard_normal((20, 256)).astype(np.float16)).to(device)
    w = torch.from_numpy((rng.standard_normal((136, 256)) * 0.05).astype(np.float16)).to(device)
    f32 = ep in (_lib.EPILOGUE_STORE_F32, _lib.EPILOGUE_ADD_F32)
    start = torch.from_numpy(rng.standard_normal((20, 136)).astype(np.float32)).to(device)
    outs = []
    for n in ((136, 130) if silu else (132, 130)):
        cols = n // 2 if silu else n
        c = start[:, :cols].clone(memory_format=torch.contiguous_format) if f32 else \
            torch.empty((20, cols), dtype=torch.float16, device=device)
        K.gemv(a, w[:n].contiguous(), c, ep)
        outs.append(c[:, :64 if silu else 128])
    torch.cuda.synchronize()
    view = torch.int32 if f32 else torch.int16
    assert torch.equal(outs[0].view(view), outs[1].view(view))


@pytest.mark.parametrize("R,hidden", [(1, 2048), (32, 2048), (5, 1000), (4, 1002), (3, 4096), (2, 5120)])
def test_rmsnorm_rows_matches_oracle(device, R, hidden):
    """f16 outputs within one f16 ulp of the oracle's f32 rows (cpu_backend.cpp:34-39; the GPU's double sum of
    squares runs in another order), through a row list. Widths that are a multiple of 4 take runs of 4 adjacent
    elements per load and store, 1002 one element at a time, 5120 the form that re-reads its row."""
    rng = np.random.default_rng(R * 100 + hidden)
    x = rng.standard_normal((R + 2, hidden)).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    rows = list(range(R + 1, 1, -1))[:R]
    out = torch.full((R, hidden), float("nan"), dtype=torch.float16, device=device)
    keep = K.rmsnorm_rows(torch.from_numpy(x).to(device), torch.from_numpy(w).to(device), out, 1e-6, rows=rows)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = np.stack([oracle.rmsnorm(x[r], w, 1e-6) for r in rows])
    np.testing.assert_allclose(got, want, rtol=2.0 ** -10, atol=2.0 ** -24)
    del keep
