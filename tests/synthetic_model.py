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

H, I, NH, NKV, D = 1024, 3072, 16, 8, 128
Q, KV = NH * D, NKV * D


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
