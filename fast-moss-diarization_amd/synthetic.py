"""Seeded synthetic checkpoints in the reference's tensor naming.

Linear weights and the embedding are N(0, std^2) (std 0.02 by default).
RMSNorm gains are 1 + N(0, std^2): a gain drawn around zero would scale every
normalised activation towards zero and hide errors in the layers behind it.
Names follow Qwen3::load (qwen3.rs:355-376) under "model.language_model.".
"""
from __future__ import annotations

import numpy as np

PREFIX = "model.language_model."


def synthetic_weights(cfg, seed: int = 0, std: float = 0.02) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    H, I, hd = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    qd, kd = cfg.q_dim(), cfg.kv_dim()

    def lin(o, i):
        return (rng.standard_normal((o, i), dtype=np.float32) * np.float32(std)).astype(np.float32)

    def gain(n):
        return (1.0 + rng.standard_normal(n, dtype=np.float32) * np.float32(std)).astype(np.float32)

    w: dict[str, np.ndarray] = {}
    for li in range(cfg.num_hidden_layers):
        p = f"{PREFIX}layers.{li}."
        w[p + "self_attn.q_proj.weight"] = lin(qd, H)
        w[p + "self_attn.k_proj.weight"] = lin(kd, H)
        w[p + "self_attn.v_proj.weight"] = lin(kd, H)
        w[p + "self_attn.o_proj.weight"] = lin(H, qd)
        w[p + "mlp.gate_proj.weight"] = lin(I, H)
        w[p + "mlp.up_proj.weight"] = lin(I, H)
        w[p + "mlp.down_proj.weight"] = lin(H, I)
        w[p + "input_layernorm.weight"] = gain(H)
        w[p + "post_attention_layernorm.weight"] = gain(H)
        w[p + "self_attn.q_norm.weight"] = gain(hd)
        w[p + "self_attn.k_norm.weight"] = gain(hd)
    w[PREFIX + "embed_tokens.weight"] = lin(cfg.vocab_size, H)
    w[PREFIX + "norm.weight"] = gain(H)
    return w
