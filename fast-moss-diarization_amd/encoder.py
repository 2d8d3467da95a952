"""The audio path on the HIP library: the Whisper encoder and the VqAdaptor
(``WhisperEncoder`` / ``VqAdaptor`` / ``MossModel::encode_audio``,
crates/fmd-core/src/model/whisper_encoder.rs, adaptor.rs, mod.rs:82-126),
behind the ``fmd_enc_*`` entry points of ``include/fmd_dec.h``.

``AudioEncoder`` mirrors the reference's calls: ``forward`` is
``WhisperEncoder::forward`` (log-mel chunks (n, n_mels, frames) in, frames
(n, frames/2, d_model) out), ``merge_and_project`` is
``VqAdaptor::merge_and_project`` and ``encode_audio`` is
``MossModel::encode_audio``: every chunk through the encoder in batches of
``encoder_batch``, each chunk trimmed to its token count times the merge
size, the chunks of each audio joined in order, then merged and projected
into the decoder's hidden size.  Everything runs in the activation dtype of
the precision (int8 keeps the audio path dense in f16, whisper_encoder.rs:31-33,
adaptor.rs:27-29).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from .decoder import (FmdAudioConfig, FmdError, Precision, _as_src, _check, _data_ptr, _ptr,
                      lib)

ENC = "model.whisper_encoder."
ADA = "model.vq_adaptor."
DEFAULT_ENCODER_BATCH = 16  # mod.rs:19-23


@dataclass(frozen=True)
class AudioConfig:
    """AudioConfig (config.rs:60-75) plus the adaptor widths that
    MossModel::load passes (mod.rs:47-53): adaptor_input_dim (= d_model *
    audio_merge_size), the decoder's hidden size and its rms_norm_eps, which
    is the adaptor LayerNorm's eps."""

    num_mel_bins: int = 80
    d_model: int = 1024
    encoder_layers: int = 24
    encoder_attention_heads: int = 16
    encoder_ffn_dim: int = 4096
    max_source_positions: int = 1500
    adaptor_input_dim: int = 4096
    hidden_size: int = 1024
    audio_merge_size: int = 4
    norm_eps: float = 1e-6

    def head_dim(self) -> int:
        return self.d_model // self.encoder_attention_heads

    def frames(self) -> int:
        """Mel frames of one 30 s chunk: conv2 halves them to max_source_positions."""
        return 2 * self.max_source_positions


# Whisper-medium encoder + the VqAdaptor into Qwen3-0.6B's 1024-wide stream.
WHISPER_MEDIUM = AudioConfig()


def _c_cfg(cfg: AudioConfig) -> FmdAudioConfig:
    return FmdAudioConfig(cfg.num_mel_bins, cfg.d_model, cfg.encoder_layers,
                          cfg.encoder_attention_heads, cfg.encoder_ffn_dim,
                          cfg.max_source_positions, cfg.adaptor_input_dim, cfg.hidden_size,
                          cfg.audio_merge_size, float(cfg.norm_eps))


def audio_weight_shapes(cfg: AudioConfig) -> dict:
    """Checkpoint names and shapes of the audio path (whisper_encoder.rs:27-42,
    73-80, 118-138; adaptor.rs:18-35)."""
    d, f, m, H = cfg.d_model, cfg.encoder_ffn_dim, cfg.num_mel_bins, cfg.hidden_size
    s = {
        ENC + "conv1.weight": (d, m, 3), ENC + "conv1.bias": (d,),
        ENC + "conv2.weight": (d, d, 3), ENC + "conv2.bias": (d,),
        ENC + "embed_positions.weight": (cfg.max_source_positions, d),
        ENC + "layer_norm.weight": (d,), ENC + "layer_norm.bias": (d,),
        ADA + "layers.0.weight": (H, cfg.adaptor_input_dim), ADA + "layers.0.bias": (H,),
        ADA + "layers.2.weight": (H, H), ADA + "layers.2.bias": (H,),
        ADA + "layers.3.weight": (H,), ADA + "layers.3.bias": (H,),
    }
    for i in range(cfg.encoder_layers):
        p = ENC + f"layers.{i}."
        s.update({
            p + "self_attn.q_proj.weight": (d, d), p + "self_attn.q_proj.bias": (d,),
            p + "self_attn.k_proj.weight": (d, d),
            p + "self_attn.v_proj.weight": (d, d), p + "self_attn.v_proj.bias": (d,),
            p + "self_attn.out_proj.weight": (d, d), p + "self_attn.out_proj.bias": (d,),
            p + "self_attn_layer_norm.weight": (d,), p + "self_attn_layer_norm.bias": (d,),
            p + "fc1.weight": (f, d), p + "fc1.bias": (f,),
            p + "fc2.weight": (d, f), p + "fc2.bias": (d,),
            p + "final_layer_norm.weight": (d,), p + "final_layer_norm.bias": (d,),
        })
    return s


def synthetic_audio_weights(cfg: AudioConfig, seed: int = 0, std: float = 0.02) -> dict:
    """Seeded f32 weights for every audio-path tensor: projections and
    convolutions N(0, std^2) (conv1 scaled by 1/sqrt(3 n_mels) so its output
    stays O(1)), biases N(0, std^2), LayerNorm gains 1 + N(0, std^2),
    positions N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in audio_weight_shapes(cfg).items():
        if "norm" in name or name.startswith(ADA + "layers.3"):
            v = (1.0 + std * rng.standard_normal(shape)) if name.endswith("weight") else \
                std * rng.standard_normal(shape)
        elif "embed_positions" in name:
            v = 0.1 * rng.standard_normal(shape)
        elif name.endswith("conv1.weight"):
            v = rng.standard_normal(shape) / np.sqrt(3.0 * cfg.num_mel_bins)
        else:
            v = std * rng.standard_normal(shape)
        out[name] = v.astype(np.float32)
    return out


def synthetic_mel(n: int, cfg: AudioConfig, seed: int = 0) -> np.ndarray:
    """Log-mel-like chunks (n, n_mels, frames): Whisper's normalised log-mel
    lies in about [-1, 1.5]; uniform values in that range."""
    rng = np.random.default_rng(seed)
    return rng.uniform(-1.0, 1.5, (n, cfg.num_mel_bins, cfg.frames())).astype(np.float32)
