"""Shared helpers of the GPU parity tests: build the HIP decoder and the CPU
oracle from one synthetic checkpoint and compare their outputs."""
from __future__ import annotations

import numpy as np

TOL = {"f32": 1e-4, "f16": 2e-2, "bf16": 2e-2, "int8": 2e-2}
OPREC = {"f32": 0, "f16": 1, "bf16": 2, "int8": 3}


def tiny_cfg(fmd, layers=2, vocab=1024):
    return fmd.TextConfig(vocab_size=vocab, hidden_size=256, intermediate_size=512,
                          num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                          head_dim=128, rope_theta=1e6)


def small_cfg(fmd, layers=2, vocab=2048):
    """Full Qwen3-0.6B layer widths, fewer layers and a smaller vocabulary."""
    return fmd.TextConfig(vocab_size=vocab, hidden_size=1024, intermediate_size=3072,
                          num_hidden_layers=layers, num_attention_heads=16, num_key_value_heads=8,
                          head_dim=128, rope_theta=1e6)


def build_pair(fmd, orc, cfg, prec: str, seed=0, max_len=8192, weights=None):
    w = weights if weights is not None else fmd.synthetic_weights(cfg, seed=seed)
    gpu = fmd.Qwen3(cfg, prec, max_len=max_len).load(w)
    ref = orc.OracleModel(cfg, OPREC[prec], max_len).load(w)
    return gpu, ref, w


def storage_to_f32(a: np.ndarray, prec: str) -> np.ndarray:
    if prec == "bf16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def f32_to_storage(x: np.ndarray, prec: str, orc) -> np.ndarray:
    return orc.to_storage(x, OPREC[prec])


def top2_margin(logits: np.ndarray) -> np.ndarray:
    s = np.sort(logits, axis=-1)
    return s[..., -1] - s[..., -2]


def check_greedy(gpu_out, ref_model, prompts, budget, eos, tol, force=None, block=256):
    """Tokens must agree wherever the oracle's top-2 logit margin exceeds tol.

    Replays the oracle along the GPU's own tokens; at the first step where a
    row differs, the oracle's margin there must be <= tol (a near-tie), after
    which that row is not compared further.  Returns the number of compared
    tokens."""
    emb, pad = ref_model.padded_embeds(prompts)
    b = len(prompts)
    kv = ref_model.new_kv(b, emb.shape[1] + budget)
    logits = ref_model.prefill(kv, emb, pad, block=block)
    done = [False] * b
    diverged = [False] * b
    pos = [0] * b
    compared = 0
    for step in range(budget):
        ref_next = logits.argmax(-1)
        margins = top2_margin(logits)
        feed = []
        for i in range(b):
            toks, fin = gpu_out[i]
            if done[i] or diverged[i]:
                feed.append(eos)
                continue
            forced = force is not None and force[i] == step
            want = eos if forced else int(ref_next[i])
            have = toks[pos[i]] if pos[i] < len(toks) else eos
            if have != want:
                assert margins[i] <= tol, (
                    f"row {i} step {step}: device {have} vs oracle {want}, margin {margins[i]:.4g}")
                diverged[i] = True
                feed.append(eos)
                continue
            compared += 1
            if want == eos:
                done[i] = True
                assert fin == 1, f"row {i} should finish with Stop"
                feed.append(eos)
            else:
                pos[i] += 1
                feed.append(want)
        if all(d or v for d, v in zip(done, diverged)) or step + 1 == budget:
            break
        logits = ref_model.decode_step(kv, feed, pad)
    for i in range(b):
        if not diverged[i] and not done[i]:
            assert len(gpu_out[i][0]) == pos[i], f"row {i}: extra tokens"
    return compared
