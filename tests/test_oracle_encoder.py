"""Pins of the oracle's audio path (oracle/fmd_oracle_encoder.c) on the CPU:

- conv1d (padding 1, stride 1 and 2) against a brute-force numpy sum on tiny
  inputs, and its output lengths (3000 -> 3000 -> 1500 frames,
  whisper_encoder.rs:139-152);
- gelu_erf against math.erf, silu and LayerNorm against their closed forms
  in float64;
- the dense attention against an explicit numpy softmax, scores unscaled
  (the encoder scales q and k instead);
- the time merge of the adaptor against the reference's own tests
  (adaptor.rs:71-128: frames folded into features in order, 1500 frames into
  375 tokens, a trailing partial group dropped);
- the whole encoder and adaptor in f32 against an independent torch
  restatement built from library routines (tests/torch_encoder_ref.py), with
  the head_dim^-1/4 scaling of q and k and no k_proj bias;
- the same in bf16 against the torch twin with the same rounding points;
- encode_audio's chunk trimming and per-audio concatenation (mod.rs:82-126)
  against a restatement over the oracle's own encoder and adaptor outputs.
"""
import dataclasses
import importlib
import math

import numpy as np
import pytest
import torch

from tests.torch_encoder_ref import TorchWhisper

enc_mod = importlib.import_module("fast-moss-diarization_amd.encoder")


def tiny_audio(layers=2, **kw):
    base = dict(num_mel_bins=8, d_model=64, encoder_layers=layers, encoder_attention_heads=4,
                encoder_ffn_dim=128, max_source_positions=12, adaptor_input_dim=128,
                hidden_size=48, audio_merge_size=2, norm_eps=1e-6)
    base.update(kw)
    return enc_mod.AudioConfig(**base)


def test_conv1d_brute_force(orc):
    rng = np.random.default_rng(0)
    for stride, t in ((1, 11), (2, 11), (2, 12), (1, 1)):
        x = rng.standard_normal((2, 3, t)).astype(np.float32)
        w = rng.standard_normal((5, 3, 3)).astype(np.float32)
        got = orc.conv1d(x, w, stride)
        tout = (t + 2 - 3) // stride + 1
        want = np.zeros((2, 5, tout))
        for b in range(2):
            for o in range(5):
                for j in range(tout):
                    for c in range(3):
                        for k in range(3):
                            src = j * stride + k - 1
                            if 0 <= src < t:
                                want[b, o, j] += float(w[o, c, k]) * float(x[b, c, src])
        assert got.shape == want.shape
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    # Whisper's window: 3000 mel frames -> 3000 -> 1500 positions
    assert (3000 + 2 - 3) // 1 + 1 == 3000 and (3000 + 2 - 3) // 2 + 1 == 1500


def test_gelu_silu_layernorm_closed_forms(orc):
    x = np.linspace(-6, 6, 1001).astype(np.float32)
    g = orc.gelu_erf(x)
    want = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    np.testing.assert_allclose(g, want, rtol=2e-6, atol=2e-7)
    # the tanh approximation is not what gelu_erf computes
    tanh = 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))
    assert np.max(np.abs(g - tanh)) > 1e-4
    s = orc.silu(x)
    np.testing.assert_allclose(s, x / (1 + np.exp(-x.astype(np.float64))), rtol=2e-6, atol=1e-7)
    rng = np.random.default_rng(1)
    a = (rng.standard_normal((7, 48)) * 3 + 2).astype(np.float32)
    w = rng.standard_normal(48).astype(np.float32)
    b = rng.standard_normal(48).astype(np.float32)
    y = orc.layernorm(a, w, b, 1e-5)
    a64 = a.astype(np.float64)
    mu = a64.mean(-1, keepdims=True)
    var = ((a64 - mu) ** 2).mean(-1, keepdims=True)
    np.testing.assert_allclose(y, (a64 - mu) / np.sqrt(var + 1e-5) * w + b, rtol=1e-5, atol=1e-5)
    # bf16 rounding of the output only
    yb = orc.layernorm(a, w, b, 1e-5, orc.BF16)
    np.testing.assert_array_equal(yb, orc.round_to(y, orc.BF16))


def test_dense_attention_unscaled_softmax(orc):
    rng = np.random.default_rng(2)
    t, heads, hd = 9, 3, 8
    q, k, v = (rng.standard_normal((t, heads * hd)).astype(np.float32) for _ in range(3))
    got = orc.attention_dense(q, k, v, heads)
    want = np.zeros((t, heads * hd))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl].astype(np.float64) @ k[:, sl].T.astype(np.float64)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        want[:, sl] = p @ v[:, sl]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def _identity_adaptor(cfg):
    """Adaptor weights whose fc1 and fc2 pass the merged row through (before
    silu and LayerNorm)."""
    w = {}
    H, n = cfg.hidden_size, cfg.adaptor_input_dim
    w1 = np.zeros((H, n), np.float32)
    w1[np.arange(min(H, n)), np.arange(min(H, n))] = 1.0
    w[enc_mod.ADA + "layers.0.weight"] = w1
    w[enc_mod.ADA + "layers.0.bias"] = np.zeros(H, np.float32)
    w[enc_mod.ADA + "layers.2.weight"] = np.eye(H, dtype=np.float32)
    w[enc_mod.ADA + "layers.2.bias"] = np.zeros(H, np.float32)
    w[enc_mod.ADA + "layers.3.weight"] = np.ones(H, np.float32)
    w[enc_mod.ADA + "layers.3.bias"] = np.zeros(H, np.float32)
    return w


def _with_adaptor(cfg, ada, seed=0):
    w = enc_mod.synthetic_audio_weights(cfg, seed)
    w.update(ada)
    return w


def test_time_merge_known_answers(orc):
    """adaptor.rs:71-128: (1, 4, 2) frames 0..7 merge (size 4) into one row
    0..7; 1500 frames merge into 375 rows; 7 frames at merge 4 give 1 row."""
    cfg = tiny_audio(d_model=64, audio_merge_size=4, adaptor_input_dim=256, hidden_size=256)
    e = orc.OracleEncoder(cfg, orc.F32).load(_with_adaptor(cfg, _identity_adaptor(cfg)))
    frames = np.zeros((4, 64), np.float32)
    frames[:, :2] = np.arange(8, dtype=np.float32).reshape(4, 2)
    out = e.adaptor(frames)
    assert out.shape == (1, 256)
    # the merged row is frames 0..3 back to back: features 0,1 of frame f at
    # columns 64 f, 64 f + 1
    merged = frames.reshape(-1)
    h = merged / (1 + np.exp(-merged.astype(np.float64)))
    mu, var = h.mean(), h.var()
    np.testing.assert_allclose(out[0], (h - mu) / np.sqrt(var + 1e-6), rtol=1e-4, atol=1e-5)
    assert [float(merged[64 * f + j]) for f in range(4) for j in range(2)] == list(range(8))
    assert e.adaptor(np.zeros((7, 64), np.float32)).shape == (1, 256)
    assert e.adaptor(np.zeros((1500, 64), np.float32)).shape == (375, 256)


@pytest.mark.parametrize("prec", ["f32", "bf16"])
def test_encoder_and_adaptor_against_torch(orc, prec):
    cfg = tiny_audio(layers=2)
    w = enc_mod.synthetic_audio_weights(cfg, seed=3)
    p = orc.F32 if prec == "f32" else orc.BF16
    e = orc.OracleEncoder(cfg, p).load(w)
    ref = TorchWhisper(cfg, w, torch.float32 if prec == "f32" else torch.bfloat16)
    mel = np.random.default_rng(4).uniform(-1, 1.5, (2, cfg.num_mel_bins, 24)).astype(np.float32)
    got = e.forward(mel)
    with torch.no_grad():
        want = ref.forward(mel).numpy()
    assert got.shape == (2, 12, cfg.d_model)
    if prec == "f32":
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)
    else:
        # same rounding points, different f32 summation order: a few values
        # may sit one bf16 step apart, nothing more
        d = np.abs(got - want)
        assert d.max() <= 2 * 2.0 ** -7 * max(1.0, float(np.abs(want).max()))
        assert np.mean(d > 0) < 0.1
    stem = e.stem(mel)
    with torch.no_grad():
        np.testing.assert_allclose(stem, ref.stem(mel).numpy(), rtol=1e-4 if prec == "f32" else 1e-2,
                                   atol=1e-4 if prec == "f32" else 1e-2)
    frames = got[0]
    a = e.adaptor(frames)
    with torch.no_grad():
        aw = ref.adaptor(frames).numpy()
    assert a.shape == (6, cfg.hidden_size)
    tol = 1e-4 if prec == "f32" else 3e-2
    np.testing.assert_allclose(a, aw, rtol=tol, atol=tol)


def test_qk_scaling_is_per_operand(orc):
    """q and k are each scaled by head_dim^-1/4 (whisper_encoder.rs:53-56): in
    bf16, scaling the product by head_dim^-1/2 instead rounds differently, and
    the torch twin that scales each operand agrees with the oracle more
    closely than one that scales the product."""
    cfg = tiny_audio(layers=1, encoder_attention_heads=2)   # head_dim 32
    w = enc_mod.synthetic_audio_weights(cfg, seed=9, std=0.2)
    e = orc.OracleEncoder(cfg, orc.BF16).load(w)
    mel = np.random.default_rng(10).uniform(-1, 1.5, (3, cfg.num_mel_bins, 24)).astype(np.float32)
    got = e.forward(mel)
    twin = TorchWhisper(cfg, w, torch.bfloat16)
    with torch.no_grad():
        good = twin.forward(mel).numpy()

    class ProductScaled(TorchWhisper):
        def layer(self, i, x):
            # scale the product once by head_dim^-1/2 instead of q and k
            saved = {}
            p = enc_mod.ENC + f"layers.{i}."
            for nm in ("self_attn.q_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.weight"):
                saved[nm] = self.w[p + nm]
            hd = self.cfg.d_model // self.cfg.encoder_attention_heads
            self.w[p + "self_attn.q_proj.weight"] = saved["self_attn.q_proj.weight"] * hd ** -0.25
            self.w[p + "self_attn.q_proj.bias"] = saved["self_attn.q_proj.bias"] * hd ** -0.25
            self.w[p + "self_attn.k_proj.weight"] = saved["self_attn.k_proj.weight"] * hd ** -0.25
            try:
                return super().layer(i, x)
            finally:
                self.w.update({p + k: v for k, v in saved.items()})

    with torch.no_grad():
        bad = ProductScaled(cfg, w, torch.bfloat16).forward(mel).numpy()
    assert np.mean(np.abs(got - good)) < np.mean(np.abs(got - bad))


def test_encode_audio_reassembly(orc):
    """mod.rs:82-126: chunk i keeps chunk_token_lengths[i] * merge frames; the
    kept frames of each audio are joined in chunk order, then merged and
    projected; a chunk asking for more frames than it has keeps all."""
    cfg = tiny_audio(layers=1)
    e = orc.OracleEncoder(cfg, orc.F32).load(enc_mod.synthetic_audio_weights(cfg, seed=5))
    mel = np.random.default_rng(6).uniform(-1, 1.5, (4, cfg.num_mel_bins, 24)).astype(np.float32)
    tokens = [6, 2, 3, 9]      # 12 frames per chunk, merge 2: 9 tokens -> all 12 frames
    mapping = [1, 0, 1, 2]
    got = e.encode_audio(mel, tokens, mapping, 3)
    frames = e.forward(mel)
    for a in range(3):
        parts = [frames[i, :min(tokens[i] * 2, 12)] for i in range(4) if mapping[i] == a]
        want = e.adaptor(np.concatenate(parts, 0))
        np.testing.assert_array_equal(got[a], want)
    assert [g.shape[0] for g in got] == [2, 6 + 3, 6]


def test_audio_weight_names_cover_the_oracle(orc):
    cfg = tiny_audio(layers=3)
    w = enc_mod.synthetic_audio_weights(cfg, seed=1)
    e = orc.OracleEncoder(cfg, orc.F32)
    missing = dict(w)
    missing.pop(enc_mod.ENC + "layers.2.fc2.bias")
    with pytest.raises(AssertionError):
        e.load(missing)
    with pytest.raises(orc.OracleError):
        orc.OracleEncoder(cfg, orc.F32).load({enc_mod.ENC + "layers.0.self_attn.k_proj.bias":
                                              np.zeros(64, np.float32)})
    assert dataclasses.replace(cfg, encoder_layers=24) == tiny_audio(layers=24)
