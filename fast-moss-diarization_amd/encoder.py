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


_MEL_CODES = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.uint16): 2}


def _mel_src(mel):
    """(dtype code, on_device, shape, keepalive) of log-mel chunks."""
    if isinstance(mel, np.ndarray):
        a = np.ascontiguousarray(mel)
        if a.dtype not in _MEL_CODES:
            a = a.astype(np.float32)
        return _MEL_CODES[a.dtype], 0, a.shape, a
    return _as_src(mel)


class AudioEncoder:
    """WhisperEncoder + VqAdaptor (whisper_encoder.rs, adaptor.rs) on one
    MI355X; the activation dtype follows the precision (int8 -> f16)."""

    def __init__(self, cfg: AudioConfig = WHISPER_MEDIUM,
                 precision: Precision | str = Precision.BF16, device: int = 0):
        self.cfg = cfg
        self.precision = Precision.parse(precision) if isinstance(precision, str) else Precision(precision)
        h = ctypes.c_void_p()
        c = _c_cfg(cfg)
        _check(lib().fmd_enc_create(ctypes.byref(c), int(self.precision), device, ctypes.byref(h)))
        self.handle = h
        self.act_np = np.float32 if self.precision == Precision.F32 else (
            np.uint16 if self.precision == Precision.BF16 else np.float16)

    def __del__(self):
        if getattr(self, "handle", None):
            lib().fmd_enc_destroy(self.handle)
            self.handle = None

    # -- loading ----------------------------------------------------------
    def set_weight(self, name: str, tensor) -> None:
        code, on_dev, shape, keep = _as_src(tensor)
        shp = (ctypes.c_int64 * len(shape))(*shape)
        _check(lib().fmd_enc_set_weight(self.handle, name.encode(), code, shp, len(shape),
                                        _data_ptr(keep), on_dev))

    def load(self, tensors: dict) -> "AudioEncoder":
        for name, t in tensors.items():
            self.set_weight(name, t)
        if not self.ready():
            raise FmdError(-2, "audio weights are incomplete")
        return self

    def ready(self) -> bool:
        return bool(lib().fmd_enc_ready(self.handle))

    def set_stream(self, stream_handle: int | None) -> None:
        _check(lib().fmd_enc_set_stream(self.handle, stream_handle))

    # -- forward ------------------------------------------------------------
    def forward(self, mel) -> np.ndarray:
        """WhisperEncoder::forward: (n, n_mels, frames) -> (n, frames/2, d_model)
        in the activation dtype's storage (bf16 as uint16 bits)."""
        code, on_dev, shape, keep = _mel_src(mel)
        n, _, frames = shape
        out = np.empty((n, frames // 2, self.cfg.d_model), dtype=self.act_np)
        _check(lib().fmd_enc_forward(self.handle, _data_ptr(keep), code, on_dev, n, frames,
                                     _ptr(out), 0))
        return out

    def forward_device(self, mel, out_ptr: int) -> None:
        """forward into a device buffer of (n, frames/2, d_model) activation values."""
        code, on_dev, shape, keep = _mel_src(mel)
        n, _, frames = shape
        _check(lib().fmd_enc_forward(self.handle, _data_ptr(keep), code, on_dev, n, frames,
                                     out_ptr, 1))

    def layers(self, x: np.ndarray, first: int, n: int, final_norm: bool = False) -> np.ndarray:
        """Encoder layers [first, first + n) (and the final LayerNorm) on
        hidden states (windows, t, d_model) in the activation dtype's storage."""
        a = np.ascontiguousarray(x, dtype=self.act_np)
        w, t, _ = a.shape
        out = np.empty_like(a)
        _check(lib().fmd_enc_layers(self.handle, _ptr(a), 0, w, t, first, n, int(final_norm),
                                    _ptr(out), 0))
        return out

    def merge_and_project(self, frames: np.ndarray) -> np.ndarray:
        """VqAdaptor::merge_and_project of one audio's frames (rows, d_model)."""
        a = np.ascontiguousarray(frames, dtype=self.act_np)
        g = a.shape[0] // self.cfg.audio_merge_size
        out = np.empty((g, self.cfg.hidden_size), dtype=self.act_np)
        if g:
            _check(lib().fmd_enc_adaptor(self.handle, _ptr(a), 0, a.shape[0], _ptr(out), 0))
        return out

    def encode_offsets(self, chunk_tokens: Sequence[int], chunk_mapping: Sequence[int],
                       num_audios: int, frames: int) -> np.ndarray:
        """Rows of each audio's embeddings (the size query of encode_audio)."""
        ct = np.ascontiguousarray(np.asarray(chunk_tokens, dtype=np.int32))
        cm = np.ascontiguousarray(np.asarray(chunk_mapping, dtype=np.int32))
        offs = np.zeros(num_audios + 1, dtype=np.int64)
        _check(lib().fmd_enc_encode_audio(self.handle, None, 0, 0, len(ct), frames, _ptr(ct),
                                          _ptr(cm), num_audios, 1, None, 0, _ptr(offs)))
        return offs

    def encode_audio(self, mel, chunk_tokens: Sequence[int], chunk_mapping: Sequence[int],
                     num_audios: int, encoder_batch: int = DEFAULT_ENCODER_BATCH) -> list:
        """MossModel::encode_audio (mod.rs:82-126): one (tokens, hidden) array
        per audio, in the activation dtype's storage."""
        code, on_dev, shape, keep = _mel_src(mel)
        n, _, frames = shape
        ct = np.ascontiguousarray(np.asarray(chunk_tokens, dtype=np.int32))
        cm = np.ascontiguousarray(np.asarray(chunk_mapping, dtype=np.int32))
        if len(ct) != n or len(cm) != n:
            raise FmdError(-1, "one token length and one audio index per chunk")
        offs = self.encode_offsets(ct, cm, num_audios, frames)
        out = np.empty((max(int(offs[-1]), 1), self.cfg.hidden_size), dtype=self.act_np)
        _check(lib().fmd_enc_encode_audio(self.handle, _data_ptr(keep), code, on_dev, n, frames,
                                          _ptr(ct), _ptr(cm), num_audios, encoder_batch,
                                          _ptr(out), 0, _ptr(offs)))
        return [out[offs[a]:offs[a + 1]] for a in range(num_audios)]
