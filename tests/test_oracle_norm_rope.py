"""Pins the oracle's QK-RMSNorm, rotary frequencies and rotate-half RoPE
(src/backend/cpu/cpu_backend.cpp:34-39, :85-88, :262-272) against the
transformers library's Qwen3 modules (the implementation the reference's own
goldens come from, reference/golden.py) and against closed forms."""
import numpy as np
import pytest
import torch
from transformers import Qwen3Config
from transformers.models.qwen3 import modeling_qwen3 as mq

import oracle

D = 128
THETA = 1e6


def _hf_rotary():
    cfg = Qwen3Config(hidden_size=1024, num_attention_heads=16, num_key_value_heads=8, head_dim=D, rope_theta=THETA,
                      max_position_embeddings=40960)
    return mq.Qwen3RotaryEmbedding(cfg)


def test_inv_freq_matches_transformers():
    got = oracle.inv_freq(THETA, D)
    want = _hf_rotary().inv_freq.numpy()
    assert got.dtype == np.float32 and got.shape == (D // 2,)
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)
    assert got[0] == 1.0


def test_rmsnorm_matches_transformers(rng):
    norm = mq.Qwen3RMSNorm(D, eps=1e-6)
    for scale in (1.0, 1e-3, 300.0):
        x = (rng.standard_normal((64, D)) * scale).astype(np.float32)
        w = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
        with torch.no_grad():
            norm.weight.copy_(torch.from_numpy(w))
            want = norm(torch.from_numpy(x)).numpy()
        got = np.stack([oracle.rmsnorm(r, w, 1e-6) for r in x])
        np.testing.assert_allclose(got, want, rtol=3e-6, atol=1e-7)


def test_rmsnorm_unit_weight_gives_unit_rms(rng):
    x = (rng.standard_normal(D) * 7).astype(np.float32)
    y = oracle.rmsnorm(x, np.ones(D, np.float32), 0.0)
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 1e-6
    # eps matters when the input is tiny: rms = sqrt(ss/n) / sqrt(ss/n + eps)
    t = np.full(D, 1e-4, np.float32)
    y = oracle.rmsnorm(t, np.ones(D, np.float32), 1e-6)
    np.testing.assert_allclose(y, 1e-4 / np.sqrt(1e-8 + 1e-6), rtol=1e-6)


@pytest.mark.parametrize("pos", [0, 1, 7, 511, 4095, 16383, 40959])
def test_rope_matches_transformers(rng, pos):
    rot = _hf_rotary()
    inv = oracle.inv_freq(THETA, D)
    x = rng.standard_normal((2, D)).astype(np.float32)
    t = torch.from_numpy(x).view(1, 2, 1, D)  # [batch, heads, seq, dim]
    cos, sin = rot(t, torch.tensor([[pos]]))
    want_q, _ = mq.apply_rotary_pos_emb(t, t, cos, sin, unsqueeze_dim=1)
    got = np.stack([oracle.rope(r, pos, inv) for r in x])
    # f32 angles up to 4e4 rad: both sides round pos * inv_freq the same way, cos/sin within an ulp or two.
    np.testing.assert_allclose(got, want_q.view(2, D).numpy(), rtol=0, atol=2e-5 * max(1, np.abs(x).max()))


def test_rope_closed_forms(rng):
    inv = oracle.inv_freq(THETA, D)
    x = rng.standard_normal(D).astype(np.float32)
    assert np.array_equal(oracle.rope(x, 0, inv), x)  # position 0 is the identity
    for pos in (3, 1000):
        y = oracle.rope(x, pos, inv)
        # rotate-half pairs (x_i, x_{i+64}) are rotated by pos * inv_freq[i]: a complex multiplication
        z = (x[:64].astype(np.float64) + 1j * x[64:]) * np.exp(1j * (np.float32(pos) * inv).astype(np.float64))
        np.testing.assert_allclose(y[:64], z.real, atol=2e-5)
        np.testing.assert_allclose(y[64:], z.imag, atol=2e-5)
        # pair norms are kept
        np.testing.assert_allclose(np.hypot(y[:64], y[64:]), np.hypot(x[:64], x[64:]), rtol=1e-5)


def test_dot_is_an_f32_dot(rng):
    for n in (128, 7, 16, 24, 200):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        want = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        assert abs(oracle.dot(a, b) - want) <= 1e-5 * np.sqrt(n) * (np.abs(a) @ np.abs(b)) / n + 1e-6
