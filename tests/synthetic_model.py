"""A synthetic Qwen3-shaped model directory for the backend tests.

Config 1's Qwen3-0.6B attention shape (hidden 1024, 16 q / 8 kv heads, head_dim 128, QK-RMSNorm, RoPE theta 1e6)
with the 0.6B model's MLP (intermediate 3072), `layers` layers and a tied vocabulary of `vocab` tokens; N(0, 0.02)
weights written with the safetensors package in three dtypes (F32 q/k/v, BF16 gate/up, F16 the rest) so the
backend's load-time conversions are exercised. Returns the oracle's copies of the weights as the backend holds
them: f16 matrices (q/k/v concatenated, gate/up interleaved row by row) and f32 norms.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

import oracle

H, I, NH, NKV, D = 1024, 3072, 16, 8, 128
Q, KV = NH * D, NKV * D
PAGE = 16


def write_model(d: Path, layers: int = 4, vocab: int = 8192, seed: int = 20261005) -> dict:
    from safetensors.torch import save_file

    cfg = dict(model_type="qwen3", vocab_size=vocab, hidden_size=H, intermediate_size=I, num_hidden_layers=layers,
               num_attention_heads=NH, num_key_value_heads=NKV, head_dim=D, rms_norm_eps=1e-6, rope_theta=1e6,
               max_position_embeddings=2048, tie_word_embeddings=True, eos_token_id=2)
    g = torch.Generator().manual_seed(seed)
    n = lambda *s: torch.randn(*s, generator=g) * 0.02  # noqa: E731
    ones = lambda k: 1 + 0.1 * torch.randn(k, generator=g)  # noqa: E731
    t = {"model.embed_tokens.weight": n(vocab, H).to(torch.float16), "model.norm.weight": ones(H)}
    for layer in range(layers):
        p = f"model.layers.{layer}."
        t[p + "self_attn.q_proj.weight"] = n(Q, H)
        t[p + "self_attn.k_proj.weight"] = n(KV, H)
        t[p + "self_attn.v_proj.weight"] = n(KV, H)
        t[p + "self_attn.o_proj.weight"] = n(H, Q).to(torch.float16)
        t[p + "mlp.gate_proj.weight"] = n(I, H).to(torch.bfloat16)
        t[p + "mlp.up_proj.weight"] = n(I, H).to(torch.bfloat16)
        t[p + "mlp.down_proj.weight"] = n(H, I).to(torch.float16)
        t[p + "input_layernorm.weight"] = ones(H)
        t[p + "post_attention_layernorm.weight"] = ones(H)
        t[p + "self_attn.q_norm.weight"] = ones(D)
        t[p + "self_attn.k_norm.weight"] = ones(D)
    d.mkdir(parents=True, exist_ok=True)
    save_file({k: v.contiguous() for k, v in t.items()}, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps(cfg))
    f16 = lambda k: t[k].to(torch.float16).numpy()  # noqa: E731  (round to nearest f16, as the backend converts)
    f32 = lambda k: t[k].float().numpy()  # noqa: E731
    w = {"embed": f16("model.embed_tokens.weight"), "norm": f32("model.norm.weight"), "layers": []}
    for layer in range(layers):
        p = f"model.layers.{layer}."
        gu = np.empty((2 * I, H), np.float16)
        gu[0::2], gu[1::2] = f16(p + "mlp.gate_proj.weight"), f16(p + "mlp.up_proj.weight")
        w["layers"].append(dict(
            qkv=np.concatenate([f16(p + "self_attn.q_proj.weight"), f16(p + "self_attn.k_proj.weight"),
                                f16(p + "self_attn.v_proj.weight")]),
            o=f16(p + "self_attn.o_proj.weight"), gate_up=gu, down=f16(p + "mlp.down_proj.weight"),
            in_norm=f32(p + "input_layernorm.weight"), post_norm=f32(p + "post_attention_layernorm.weight"),
            q_norm=f32(p + "self_attn.q_norm.weight"), k_norm=f32(p + "self_attn.k_norm.weight")))
    return w


class OracleModel:
    """The forward pass composed from the oracle's pieces (rmsnorm, linear, append, attention) with the GPU path's f16
    roundings (xn, qkv, attention output and the MLP activation stored as f16; cuda_backend.cu:350-366), f16 K/V
    pages in the oracle's own pool. `w` is write_model's return value."""

    def __init__(self, w, num_blocks=64):
        self.w, self.NB = w, num_blocks
        self.k = [np.zeros((num_blocks, NKV, PAGE, D), np.uint16) for _ in w["layers"]]
        self.v = [np.zeros_like(self.k[0]) for _ in w["layers"]]
        self.inv = oracle.inv_freq(1e6, D)

    def _norm(self, h, wt):
        return np.stack([oracle.rmsnorm(r, wt, 1e-6) for r in h]).astype(np.float16)

    def forward(self, tokens, positions, table, logit_rows):
        T = len(tokens)
        h = self.w["embed"][np.asarray(tokens)].astype(np.float32)
        qs = np.array([0, T], np.int32)
        for layer, lw in enumerate(self.w["layers"]):
            xn = self._norm(h, lw["in_norm"])
            qkv = oracle.linear(xn, lw["qkv"], 0, threads=16).astype(np.float16).astype(np.float32)
            q = oracle.append_layer(qkv, positions, qs, table, self.k[layer], self.v[layer], n_heads=NH, n_kv=NKV,
                                    inv_freq_=self.inv, eps=1e-6, q_norm=lw["q_norm"], k_norm=lw["k_norm"],
                                    num_blocks=self.NB, kv_f16=True)
            att = oracle.attention_layer(q, positions, qs, table, self.k[layer], self.v[layer], n_heads=NH, n_kv=NKV,
                                         num_blocks=self.NB, kv_f16=True, q_f16=True, threads=16)
            h = oracle.linear(att.reshape(T, Q).astype(np.float16), lw["o"], 2, h, threads=16)
            xn = self._norm(h, lw["post_norm"])
            act = oracle.linear(xn, lw["gate_up"], 3, threads=16).astype(np.float16)
            h = oracle.linear(act, lw["down"], 2, h, threads=16)
        xn = self._norm(h[np.asarray(logit_rows)], self.w["norm"])
        return oracle.linear(xn, self.w["embed"], 1, threads=16)
