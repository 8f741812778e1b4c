"""Pins the oracle's slot mapping, append and causal paged attention
(src/backend/cpu/cpu_backend.cpp:155-198, :256-260) against structural
invariants, a float64 textbook reference, torch's SDPA and closed forms."""
import numpy as np
import pytest
import torch

import oracle
from helpers import D, PAGE, attention_f64, dense_kv, make_step, rel_err

H, KVH = 16, 8


def test_cache_offset_is_a_bijection_onto_table_pages(rng):
    NB, L, S, W = 12, 2, 3, 3
    tables = rng.permutation(NB)[: S * W].reshape(S, W).astype(np.int32)
    seen = {}
    for layer in range(L):
        for s in range(S):
            for kvh in range(KVH):
                for pos in range(W * PAGE):
                    off = oracle.cache_offset(tables, NB, KVH, D, s, layer, kvh, pos)
                    assert 0 <= off <= L * NB * KVH * PAGE * D - D and off % D == 0
                    assert off not in seen
                    seen[off] = (layer, s, kvh, pos)
                    # layout [layer][block][kv_head][slot][dim]
                    blk, rest = divmod(off - layer * NB * KVH * PAGE * D, KVH * PAGE * D)
                    assert blk == tables[s, pos // PAGE]
                    assert divmod(rest, PAGE * D) == (kvh, (pos % PAGE) * D)


@pytest.mark.parametrize("kv_f16", [False, True])
def test_append_writes_exactly_the_token_slots(rng, kv_f16):
    NB = 40
    step = make_step(rng, [37, 5, 64], [37, 2, 16], NB)
    dt = np.uint16 if kv_f16 else np.float32
    sentinel = np.array(0x7e01 if kv_f16 else np.nan, dtype=dt) if kv_f16 else np.float32(np.nan)
    k = np.full((NB, KVH, PAGE, D), sentinel, dtype=dt)
    v = k.copy()
    qkv = rng.standard_normal((step.T, (H + 2 * KVH) * D)).astype(np.float32)
    inv = oracle.inv_freq(1e6, D)
    oracle.append_layer(qkv, step.positions, step.query_start, step.tables, k, v, n_heads=H, n_kv=KVH, inv_freq_=inv,
                        q_norm=np.ones(D, np.float32), k_norm=np.ones(D, np.float32), num_blocks=NB, kv_f16=kv_f16)
    written = ~np.isnan(k.view(np.float16) if kv_f16 else k).all(axis=3)  # [NB, KVH, 16]
    want = np.zeros_like(written)
    for t in range(step.T):
        s, p = step.token_seq[t], step.positions[t]
        want[step.tables[s, p // PAGE], :, p % PAGE] = True
    assert np.array_equal(written, want)
    # V is stored raw (no norm, no rotation); f16 values are clamped then rounded.
    vsrc = qkv[:, (H + KVH) * D:].reshape(step.T, KVH, D)
    for t in range(step.T):
        s, p = step.token_seq[t], step.positions[t]
        row = v[step.tables[s, p // PAGE], :, p % PAGE]
        expect = vsrc[t].astype(np.float16).view(np.uint16) if kv_f16 else vsrc[t]
        assert np.array_equal(row, expect)


@pytest.mark.parametrize("kv_f16", [False, True])
def test_append_k_at_position_zero_is_each_heads_unit_rms_vector(rng, kv_f16):
    """A direct pin of the stored K (and of q): at position 0 the rotation is the identity, so with unit norm
    weights the oracle stores k = x / sqrt(mean(x^2) + eps) of its own kv head (cpu_backend.cpp:34-39, :163-170).
    Every head's source gets its own scale, so a wrong head offset fails; computed here in float64."""
    NB, eps = 4, 1e-6
    tables = np.array([[2]], np.int32)
    qkv = rng.standard_normal((1, (H + 2 * KVH) * D)) * np.repeat(np.arange(1, H + 2 * KVH + 1), D)[None, :]
    qkv = qkv.astype(np.float32)
    dt = np.uint16 if kv_f16 else np.float32
    k = np.zeros((NB, KVH, PAGE, D), dt)
    v = np.zeros_like(k)
    q = oracle.append_layer(qkv, [0], [0, 1], tables, k, v, n_heads=H, n_kv=KVH, inv_freq_=oracle.inv_freq(1e6, D),
                            eps=eps, q_norm=np.ones(D, np.float32), k_norm=np.ones(D, np.float32), num_blocks=NB,
                            kv_f16=kv_f16)
    heads = qkv[0].astype(np.float64).reshape(H + 2 * KVH, D)
    unit = heads / np.sqrt((heads ** 2).mean(axis=1, keepdims=True) + eps)
    got_k = k[2, :, 0].view(np.float16).astype(np.float64) if kv_f16 else k[2, :, 0].astype(np.float64)
    np.testing.assert_allclose(got_k, unit[H:H + KVH], rtol=1e-3 if kv_f16 else 1e-6, atol=1e-3 if kv_f16 else 1e-7)
    np.testing.assert_allclose(q[0], unit[:H], rtol=1e-6, atol=1e-7)
    assert not k[[0, 1, 3]].any() and not k[2, :, 1:].any()  # nothing else written


@pytest.mark.parametrize("kv_f16", [False, True])
def test_append_keeps_the_sign_of_zero_without_a_bias(kv_f16):
    """Without a bias the reference copies V into the cache as it is (the memcpy at cpu_backend.cpp:169; the bias
    is added only for qkv_bias models, :146-154), so a -0.0 input stays -0.0; with a bias, -0.0 + 0.0 is +0.0."""
    NB = 2
    tables = np.array([[1]], np.int32)
    qkv = np.zeros((1, (H + 2 * KVH) * D), np.float32)
    qkv[0, (H + KVH) * D:] = -0.0
    qkv[0, (H + KVH) * D + 5] = 1.5
    dt = np.uint16 if kv_f16 else np.float32
    for bias, neg_zero in ((None, True), (np.zeros((H + 2 * KVH) * D, np.float32), False)):
        k = np.zeros((NB, KVH, PAGE, D), dt)
        v = np.zeros_like(k)
        oracle.append_layer(qkv, [3], [0, 1], tables, k, v, n_heads=H, n_kv=KVH, inv_freq_=oracle.inv_freq(1e6, D),
                            bias=bias, num_blocks=NB, kv_f16=kv_f16)
        row = v[1, 0, 3].view(np.uint16 if kv_f16 else np.uint32)
        sign = 0x8000 if kv_f16 else 0x80000000
        assert row[5] == (0x3E00 if kv_f16 else np.float32(1.5).view(np.uint32))
        assert (row[[0, 1, 127]] == (sign if neg_zero else 0)).all()


def _filled(rng, step, NB, kv_f16=False, scale=1.0):
    dt = np.float32
    k = np.zeros((NB, KVH, PAGE, D), dt)
    v = np.zeros_like(k)
    for s in range(step.S):
        ctx = int(step.positions[step.query_start[s + 1] - 1]) + 1
        for pos in range(ctx):
            b = step.tables[s, pos // PAGE]
            k[b, :, pos % PAGE] = rng.standard_normal((KVH, D)) * scale
            v[b, :, pos % PAGE] = rng.standard_normal((KVH, D))
    if kv_f16:
        return oracle.f32_to_f16(k), oracle.f32_to_f16(v)
    return k, v


def test_attention_matches_float64_textbook(rng):
    NB = 200
    step = make_step(rng, [1, 17, 300, 1000], [1, 3, 1, 40], NB)
    k, v = _filled(rng, step, NB, scale=0.3)
    q = rng.standard_normal((step.T, H, D)).astype(np.float32)
    got = oracle.attention_layer(q, step.positions, step.query_start, step.tables, k, v, n_heads=H, n_kv=KVH,
                                 num_blocks=NB, kv_f16=False, threads=4)
    want = attention_f64(q, step, k, v, H, KVH)
    assert rel_err(got, want) < 1e-5


def test_attention_matches_torch_sdpa(rng):
    NB = 64
    ctx = 300
    step = make_step(rng, [ctx], [ctx], NB)  # a whole prompt: causal over itself
    k, v = _filled(rng, step, NB, scale=0.3)
    q = rng.standard_normal((step.T, H, D)).astype(np.float32)
    got = oracle.attention_layer(q, step.positions, step.query_start, step.tables, k, v, n_heads=H, n_kv=KVH,
                                 num_blocks=NB, kv_f16=False, threads=2)
    K = torch.from_numpy(dense_kv(k, step.tables[0], ctx)).double().permute(1, 0, 2)[None]  # [1, KVH, ctx, D]
    V = torch.from_numpy(dense_kv(v, step.tables[0], ctx)).double().permute(1, 0, 2)[None]
    Q = torch.from_numpy(q).double().permute(1, 0, 2)[None]                                  # [1, H, T, D]
    want = torch.nn.functional.scaled_dot_product_attention(Q, K, V, is_causal=True, enable_gqa=True)
    assert rel_err(got, want[0].permute(1, 0, 2).numpy()) < 1e-5


def test_attention_closed_forms(rng):
    NB = 16
    # ctx = 1: the output is V_0 exactly (one weight of 1.0)
    step = make_step(rng, [1], [1], NB)
    k, v = _filled(rng, step, NB)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    out = oracle.attention_layer(q, step.positions, step.query_start, step.tables, k, v, n_heads=H, n_kv=KVH,
                                 num_blocks=NB, kv_f16=False)
    b = step.tables[0, 0]
    for h in range(H):
        assert np.array_equal(out[0, h], v[b, h // 2, 0])
    # identical keys: uniform weights -> the mean of the values
    step = make_step(rng, [48], [1], NB)
    k, v = _filled(rng, step, NB)
    k[:] = k[step.tables[0, 0], :, 0][None, :, None, :]
    out = oracle.attention_layer(q, step.positions, step.query_start, step.tables, k, v, n_heads=H, n_kv=KVH,
                                 num_blocks=NB, kv_f16=False)
    mean = dense_kv(v, step.tables[0], 48).mean(axis=0)
    np.testing.assert_allclose(out[0], np.repeat(mean, 2, axis=0), rtol=1e-5, atol=1e-6)
    # one dominant key: its value
    k[:] = 0
    k[step.tables[0, 1], :, 5] = 50.0 * q[0, ::2] / np.linalg.norm(q[0, ::2], axis=1, keepdims=True)
    out = oracle.attention_layer(q, step.positions, step.query_start, step.tables, k, v, n_heads=H, n_kv=KVH,
                                 num_blocks=NB, kv_f16=False)
    for h in range(0, H, 2):
        np.testing.assert_allclose(out[0, h], v[step.tables[0, 1], h // 2, 5], rtol=1e-4, atol=1e-5)


def test_f16_storage_modes_stay_within_tolerance(rng):
    NB = 100
    step = make_step(rng, [700, 33], [1, 1], NB)
    k, v = _filled(rng, step, NB, scale=0.3)
    k16, v16 = oracle.f32_to_f16(k), oracle.f32_to_f16(v)
    q = rng.standard_normal((step.T, H, D)).astype(np.float32)
    args = (step.positions, step.query_start, step.tables)
    f32 = oracle.attention_layer(q, *args, k, v, n_heads=H, n_kv=KVH, num_blocks=NB, kv_f16=False)
    f16 = oracle.attention_layer(q, *args, k16, v16, n_heads=H, n_kv=KVH, num_blocks=NB, kv_f16=True, q_f16=True)
    assert rel_err(f16, f32) < 2e-3
