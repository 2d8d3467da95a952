"""Python facade over libfmd_dec.so, mirroring the reference decoder API.

Names and argument meanings follow crates/fmd-core/src: ``TextConfig``
(config.rs:8-58), ``Precision`` (precision.rs:10-93), ``Qwen3`` / ``KvCache``
(model/qwen3.rs:33-563) and the greedy loop of ``Engine::generate_batch``
(engine.rs:463-559).  Every call goes to the gfx950 HIP library; there is no
CPU fallback -- if the library is missing, loading fails loudly.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field
from pathlib import Path
from typing import Iterable, Sequence

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libfmd_dec.so"


class FmdError(RuntimeError):
    """A failed library call: ``code`` is the C status, the message fmd_last_error()."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class KvCacheOverflow(FmdError):
    """``kv cache overflow: {len} + {t} exceeds capacity {cap}`` (qwen3.rs:88-94)."""


FMD_ERR_OVERFLOW = -5


class _TextConfigC(ctypes.Structure):
    _fields_ = [
        ("vocab_size", ctypes.c_int32),
        ("hidden_size", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("num_hidden_layers", ctypes.c_int32),
        ("num_attention_heads", ctypes.c_int32),
        ("num_key_value_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_position_embeddings", ctypes.c_int32),
        ("rms_norm_eps", ctypes.c_double),
        ("rope_theta", ctypes.c_double),
        ("tie_word_embeddings", ctypes.c_int32),
        ("attention_bias", ctypes.c_int32),
    ]


class BatchStats(ctypes.Structure):
    """Subset of BatchStats (engine.rs:151-174) the decoder path fills."""

    _fields_ = [
        ("generate_seconds", ctypes.c_double),
        ("generated_tokens", ctypes.c_int64),
        ("micro_batches", ctypes.c_int32),
        ("prefill_seconds", ctypes.c_double),
        ("decode_seconds", ctypes.c_double),
    ]


class FmdAudioConfig(ctypes.Structure):
    """fmd_audio_config: AudioConfig (config.rs:60-75) plus the adaptor widths
    of MossModel::load (mod.rs:47-53)."""

    _fields_ = [
        ("num_mel_bins", ctypes.c_int32),
        ("d_model", ctypes.c_int32),
        ("encoder_layers", ctypes.c_int32),
        ("encoder_attention_heads", ctypes.c_int32),
        ("encoder_ffn_dim", ctypes.c_int32),
        ("max_source_positions", ctypes.c_int32),
        ("adaptor_input_dim", ctypes.c_int32),
        ("hidden_size", ctypes.c_int32),
        ("audio_merge_size", ctypes.c_int32),
        ("norm_eps", ctypes.c_double),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); these are exactly the entry points of include/fmd_dec.h
SIGNATURES = {
    "fmd_last_error": (ctypes.c_char_p, []),
    "fmd_dec_create": (_I, [ctypes.POINTER(_TextConfigC), _I, _I, _I, ctypes.POINTER(_P)]),
    "fmd_dec_destroy": (_I, [_P]),
    "fmd_dec_set_stream": (_I, [_P, _P]),
    "fmd_dec_set_spin_limit": (_I, [_P, _I]),
    "fmd_dec_stream": (_P, [_P]),
    "fmd_dec_set_weight": (_I, [_P, ctypes.c_char_p, _I, ctypes.POINTER(_I64), _I, _P, _I]),
    "fmd_dec_ready": (_I, [_P]),
    "fmd_dec_weight_bytes": (_I, [_P, ctypes.POINTER(_SZ)]),
    "fmd_dec_get_q8_0": (_I, [_P, ctypes.c_char_p, _P]),
    "fmd_quantize_q8_0": (_I, [_P, _I64, _I64, _P]),
    "fmd_kv_create": (_I, [_P, _I, _I, ctypes.POINTER(_P)]),
    "fmd_kv_destroy": (_I, [_P]),
    "fmd_kv_bytes": (_SZ, [_P, _I, _I]),
    "fmd_kv_len": (_I, [_P]),
    "fmd_kv_truncate": (_I, [_P, _I]),
    "fmd_kv_read": (_I, [_P, _I, _I, _P]),
    "fmd_kv_write": (_I, [_P, _I, _I, _P]),
    "fmd_kv_fill_random": (_I, [_P, _U64, _I]),
    "fmd_kv_set_len": (_I, [_P, _I]),
    "fmd_dec_embed": (_I, [_P, _P, _I64, _P]),
    "fmd_dec_assemble": (_I, [_P, _P, _P, _I, _P, _I, _I, _I64, _P, _P, _U32, _I, _P, _P]),
    "fmd_dec_prefill": (_I, [_P, _P, _P, _I, _P, _I, _I, _I, _P]),
    "fmd_dec_decode_step": (_I, [_P, _P, _P, _P, _I, _P]),
    "fmd_dec_generate": (_I, [_P, _P, _I, _P, _I, _I, _I, _I, _U32, _P, _P, _P, _P]),
    "fmd_dec_decode_loop": (_I, [_P, _P, _P, _P, _I, _I, _U32, _P, _P, _P, _P, _P]),
    "fmd_dec_greedy": (_I, [_P, _I, _U32, _P, _I, _P, _P, _P]),
    "fmd_engine_generate": (
        _I,
        [_P, _P, _P, _I, _I, _I, _U32, _P, _I, _P, _P, _P, _P, _P, _I,
         ctypes.POINTER(BatchStats)],
    ),
    "fmd_op_linear": (_I, [_P, _I, _I, _P, _I, _P]),
    "fmd_op_attention_decode": (_I, [_P, _P, _I, _P, _P, _I, _P]),
    "fmd_op_attention_decode_noalloc": (_I, [_P, _P, _I, _P, _P, _I, _P]),
    "fmd_op_layer_decode": (_I, [_P, _P, _I, _P, _P, _I]),
    "fmd_op_logits": (_I, [_P, _P, _I, _P]),
    "fmd_enc_create": (_I, [ctypes.POINTER(FmdAudioConfig), _I, _I, ctypes.POINTER(_P)]),
    "fmd_enc_destroy": (_I, [_P]),
    "fmd_enc_set_stream": (_I, [_P, _P]),
    "fmd_enc_set_weight": (_I, [_P, ctypes.c_char_p, _I, ctypes.POINTER(_I64), _I, _P, _I]),
    "fmd_enc_ready": (_I, [_P]),
    "fmd_enc_forward": (_I, [_P, _P, _I, _I, _I, _I, _P, _I]),
    "fmd_enc_layers": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _P, _I]),
    "fmd_enc_adaptor": (_I, [_P, _P, _I, _I, _P, _I]),
    "fmd_enc_encode_audio": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _I, _I, _P, _I, _P]),
}

_lib_handle = None


def lib() -> ctypes.CDLL:
    """Load libfmd_dec.so (built by build.py) and bind every entry point."""
    global _lib_handle
    if _lib_handle is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python {LIB_PATH.parent / 'build.py'}`"
            )
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib_handle = h
    return _lib_handle


def _check(rc: int) -> None:
    if rc != 0:
        msg = (lib().fmd_last_error() or b"").decode()
        if rc == FMD_ERR_OVERFLOW:
            raise KvCacheOverflow(rc, msg)
        raise FmdError(rc, msg)


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


class Precision(enum.IntEnum):
    """precision.rs:10-93."""

    F32 = 0
    F16 = 1
    BF16 = 2
    INT8 = 3

    @classmethod
    def parse(cls, name: str) -> "Precision":
        s = name.strip().lower().replace("-", "").replace("_", "")
        if s in ("fp32", "f32", "float32", "full"):
            return cls.F32
        if s in ("fp16", "f16", "float16", "half"):
            return cls.F16
        if s in ("bf16", "bfloat16"):
            return cls.BF16
        if s in ("int8", "i8", "q8", "q80"):
            return cls.INT8
        raise ValueError(f"unsupported dtype {s!r}")

    def activation_dtype(self) -> str:
        return {0: "f32", 1: "f16", 2: "bf16", 3: "f16"}[int(self)]

    def is_quantized(self) -> bool:
        return self is Precision.INT8

    def as_str(self) -> str:
        return {0: "fp32", 1: "fp16", 2: "bf16", 3: "int8"}[int(self)]

    @property
    def numpy_storage(self):
        """numpy dtype that holds the activation dtype's bits (bf16 as uint16)."""
        return {0: np.float32, 1: np.float16, 2: np.uint16, 3: np.float16}[int(self)]


@dataclass
class TextConfig:
    """TextConfig (config.rs:8-58) with the serde defaults of config.rs:30-41."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_position_embeddings: int = 131_072
    tie_word_embeddings: bool = False
    attention_bias: bool = False

    def q_dim(self) -> int:
        return self.num_attention_heads * self.head_dim

    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim

    def kv_repeat(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    def to_c(self) -> _TextConfigC:
        return _TextConfigC(
            self.vocab_size, self.hidden_size, self.intermediate_size, self.num_hidden_layers,
            self.num_attention_heads, self.num_key_value_heads, self.head_dim,
            self.max_position_embeddings, float(self.rms_norm_eps), float(self.rope_theta),
            int(self.tie_word_embeddings), int(self.attention_bias),
        )


# The Qwen3-0.6B decoder shape of MOSS-Transcribe-Diarize.
QWEN3_0_6B = TextConfig(
    vocab_size=151_936, hidden_size=1024, intermediate_size=3072, num_hidden_layers=28,
    num_attention_heads=16, num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6,
    rope_theta=1e6, max_position_embeddings=131_072, tie_word_embeddings=True,
)

DEFAULT_EOS = 151_645  # engine.rs:246, config.rs:111-116


class FinishReason(enum.IntEnum):
    """engine.rs:129-137."""

    LENGTH = 0
    STOP = 1


@dataclass
class Generated:
    tokens: list[int]
    finish_reason: FinishReason


class KvCache:
    """All layers' K/V caches of one micro-batch (qwen3.rs:33-108, 415-428)."""

    def __init__(self, model: "Qwen3", batch: int, capacity: int):
        self.model = model
        self.batch = batch
        self.capacity_ = capacity
        h = ctypes.c_void_p()
        _check(lib().fmd_kv_create(model.handle, batch, capacity, ctypes.byref(h)))
        self.handle = h

    def __del__(self):
        if getattr(self, "handle", None):
            lib().fmd_kv_destroy(self.handle)
            self.handle = None

    def len(self) -> int:
        return lib().fmd_kv_len(self.handle)

    def __len__(self) -> int:
        return self.len()

    def is_empty(self) -> bool:
        return self.len() == 0

    def capacity(self) -> int:
        return self.capacity_

    def truncate(self, length: int) -> None:
        _check(lib().fmd_kv_truncate(self.handle, length))

    def set_len(self, length: int) -> None:
        _check(lib().fmd_kv_set_len(self.handle, length))

    def shape(self) -> tuple[int, int, int, int]:
        c = self.model.cfg
        return (self.batch, c.num_key_value_heads, self.capacity_, c.head_dim)

    def read(self, layer: int, which: int) -> np.ndarray:
        """Layer's K (which=0) or V (which=1) as raw activation-dtype storage."""
        out = np.empty(self.shape(), dtype=self.model.precision.numpy_storage)
        _check(lib().fmd_kv_read(self.handle, layer, which, _ptr(out)))
        return out

    def write(self, layer: int, which: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data, dtype=self.model.precision.numpy_storage)
        assert data.shape == self.shape()
        _check(lib().fmd_kv_write(self.handle, layer, which, _ptr(data)))

    def fill_random(self, seed: int, length: int) -> None:
        _check(lib().fmd_kv_fill_random(self.handle, seed, length))

    @staticmethod
    def bytes_per_layer(batch: int, kv_heads: int, capacity: int, head_dim: int, esz: int) -> int:
        """KvCache::bytes_per_layer (qwen3.rs:70-78)."""
        return 2 * batch * kv_heads * capacity * head_dim * esz


def _as_src(t) -> tuple[int, int, tuple[int, ...], object]:
    """(dtype code, on_device, shape, keepalive) of a numpy array or torch tensor."""
    if isinstance(t, np.ndarray):
        a = np.ascontiguousarray(t)
        if a.dtype == np.float32:
            code = 0
        elif a.dtype == np.float16:
            code = 1
        elif a.dtype == np.uint16:  # bf16 bits
            code = 2
        else:
            a = a.astype(np.float32)
            code = 0
        return code, 0, tuple(a.shape), a
    import torch  # device tensors

    tt = t.contiguous()
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[tt.dtype]
    return code, int(tt.is_cuda), tuple(tt.shape), tt


def _data_ptr(keep) -> int:
    return keep.ctypes.data if isinstance(keep, np.ndarray) else keep.data_ptr()


class Qwen3:
    """The decoder (qwen3.rs:342-563) on one MI355X."""

    def __init__(self, cfg: TextConfig, precision: Precision | str = Precision.BF16,
                 device: int = 0, max_len: int | None = None):
        self.cfg = cfg
        self.precision = Precision.parse(precision) if isinstance(precision, str) else Precision(precision)
        # engine.rs:239-243: the RoPE table covers min(max_position_embeddings, 65536).
        self.max_len = max_len or min(cfg.max_position_embeddings, 65_536)
        h = ctypes.c_void_p()
        c = cfg.to_c()
        _check(lib().fmd_dec_create(ctypes.byref(c), int(self.precision), device, self.max_len,
                                    ctypes.byref(h)))
        self.handle = h

    def __del__(self):
        if getattr(self, "handle", None):
            lib().fmd_dec_destroy(self.handle)
            self.handle = None

    # -- loading ----------------------------------------------------------
    def set_weight(self, name: str, tensor) -> None:
        code, on_dev, shape, keep = _as_src(tensor)
        shp = (ctypes.c_int64 * len(shape))(*shape)
        _check(lib().fmd_dec_set_weight(self.handle, name.encode(), code, shp, len(shape),
                                        _data_ptr(keep), on_dev))

    def load(self, tensors: dict) -> "Qwen3":
        for name, t in tensors.items():
            self.set_weight(name, t)
        if not self.ready():
            raise FmdError(-2, "decoder weights are incomplete")
        return self

    def ready(self) -> bool:
        return bool(lib().fmd_dec_ready(self.handle))

    def weight_bytes(self) -> int:
        out = ctypes.c_size_t()
        _check(lib().fmd_dec_weight_bytes(self.handle, ctypes.byref(out)))
        return out.value

    def q8_0_blocks(self, name: str) -> np.ndarray:
        """A quantised projection's GGML block_q8_0 bytes, (rows, in/32, 34) uint8."""
        rows, cols = self._proj_shape(name)
        out = np.empty((rows, cols // 32, 34), dtype=np.uint8)
        _check(lib().fmd_dec_get_q8_0(self.handle, name.encode(), _ptr(out)))
        return out

    def _proj_shape(self, name: str) -> tuple[int, int]:
        c = self.cfg
        n = name.removeprefix("model.language_model.")
        if n in ("embed_tokens.weight", "lm_head.weight"):
            return c.vocab_size, c.hidden_size
        table = {
            "self_attn.q_proj.weight": (c.q_dim(), c.hidden_size),
            "self_attn.k_proj.weight": (c.kv_dim(), c.hidden_size),
            "self_attn.v_proj.weight": (c.kv_dim(), c.hidden_size),
            "self_attn.o_proj.weight": (c.hidden_size, c.q_dim()),
            "mlp.gate_proj.weight": (c.intermediate_size, c.hidden_size),
            "mlp.up_proj.weight": (c.intermediate_size, c.hidden_size),
            "mlp.down_proj.weight": (c.hidden_size, c.intermediate_size),
        }
        return table[n.split(".", 2)[2]]

    # -- reference API ------------------------------------------------------
    def hidden_size(self) -> int:
        return self.cfg.hidden_size

    def embed(self, ids: Sequence[int] | np.ndarray) -> np.ndarray:
        """Qwen3::embed (qwen3.rs:405-412) -> (n, hidden) activation-dtype storage."""
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32).reshape(-1))
        out = np.empty((ids.size, self.cfg.hidden_size), dtype=self.precision.numpy_storage)
        _check(lib().fmd_dec_embed(self.handle, _ptr(ids), ids.size, _ptr(out)))
        return out

    def new_caches(self, batch: int, capacity: int) -> KvCache:
        return KvCache(self, batch, capacity)

    def cache_bytes(self, batch: int, capacity: int) -> int:
        return int(lib().fmd_kv_bytes(self.handle, batch, capacity))

    def assemble(self, prompts: Sequence[Sequence[int]], audio=None, audio_token_id: int = -1,
                 total: int | None = None):
        """Device-side prompt assembly (mod.rs:128-180 splice_audio, then the
        left pad of engine.rs:476-491).  ``audio[b]`` holds row b's audio
        embeddings (n_b, hidden) as numpy or torch f32/f16/bf16, taken in order
        by its ``audio_token_id`` positions.  Returns a (B, total, hidden)
        torch tensor on the device in the activation dtype and the pad list,
        the inputs of ``prefill_device``."""
        import torch

        B = len(prompts)
        lens = [len(p) for p in prompts]
        total = int(total if total is not None else max(lens, default=0))
        ids = np.ascontiguousarray(np.concatenate([np.asarray(p, dtype=np.uint32).reshape(-1)
                                                   for p in prompts]) if B else np.zeros(0, np.uint32))
        offsets = np.zeros(B + 1, dtype=np.int64)
        offsets[1:] = np.cumsum(lens)
        hidden = self.cfg.hidden_size
        out = torch.empty((B, total, hidden), device="cuda",
                          dtype={"f32": torch.float32, "f16": torch.float16,
                                 "bf16": torch.bfloat16}[self.precision.activation_dtype()])
        pad = np.zeros(B, dtype=np.int32)
        first = np.zeros(B, dtype=np.int64)
        count = np.zeros(B, dtype=np.int64)
        rows, keep, code, on_dev, n_audio = [], None, 0, 0, 0
        if audio is not None:
            for b, a in enumerate(audio):
                if a is None:
                    continue
                first[b] = n_audio
                count[b] = a.shape[0] if a.ndim == 2 else 0
                n_audio += int(count[b])
                rows.append(a)
            if rows:
                if all(isinstance(a, np.ndarray) for a in rows):
                    cat = np.ascontiguousarray(np.concatenate([a.reshape(-1, hidden) for a in rows]))
                else:
                    cat = torch.cat([torch.as_tensor(a).reshape(-1, hidden) for a in rows]).contiguous()
                code, on_dev, _, keep = _as_src(cat)
        tid = audio_token_id if audio_token_id >= 0 else 0xFFFFFFFF
        _check(lib().fmd_dec_assemble(self.handle, _ptr(ids), _ptr(offsets), B,
                                      _data_ptr(keep) if keep is not None else None, code, on_dev,
                                      n_audio, _ptr(first), _ptr(count), tid, total,
                                      out.data_ptr(), _ptr(pad)))
        return out, pad.tolist()

    def prefill_device(self, embeds_dev, caches: KvCache, pad_lengths: Sequence[int],
                       chunk: int = 256) -> np.ndarray:
        """prefill + logits from a device (B, total, hidden) activation tensor
        such as ``assemble`` returns."""
        b, t, h = embeds_dev.shape
        pad = np.ascontiguousarray(np.asarray(pad_lengths, dtype=np.int32))
        logits = np.empty((b, self.cfg.vocab_size), dtype=np.float32)
        _check(lib().fmd_dec_prefill(self.handle, caches.handle, embeds_dev.data_ptr(), 1,
                                     _ptr(pad), b, t, chunk, _ptr(logits)))
        return logits

    def prefill(self, embeds: np.ndarray, caches: KvCache, pad_lengths: Sequence[int],
                chunk: int = 256) -> np.ndarray:
        """prefill + logits (qwen3.rs:475-496, 459-463): f32 logits (B, vocab)."""
        e = np.ascontiguousarray(embeds, dtype=self.precision.numpy_storage)
        b, t, h = e.shape
        pad = np.ascontiguousarray(np.asarray(pad_lengths, dtype=np.int32))
        logits = np.empty((b, self.cfg.vocab_size), dtype=np.float32)
        _check(lib().fmd_dec_prefill(self.handle, caches.handle, _ptr(e), 0, _ptr(pad), b, t,
                                     chunk, _ptr(logits)))
        return logits

    def decode_step(self, ids: Sequence[int], caches: KvCache,
                    pad_lengths: Sequence[int]) -> np.ndarray:
        """decode_step (qwen3.rs:499-511): f32 logits (B, vocab) at offset caches.len()."""
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32).reshape(-1))
        pad = np.ascontiguousarray(np.asarray(pad_lengths, dtype=np.int32))
        logits = np.empty((ids.size, self.cfg.vocab_size), dtype=np.float32)
        _check(lib().fmd_dec_decode_step(self.handle, caches.handle, _ptr(ids), _ptr(pad),
                                         ids.size, _ptr(logits)))
        return logits

    def generate_batch(self, prompts: Sequence[Sequence[int]], budget: int,
                       eos: int = DEFAULT_EOS, force_eot_step: Sequence[int] | None = None,
                       chunk: int = 256) -> list[Generated]:
        """Engine::generate_batch (engine.rs:463-541) for token-id prompts."""
        b = len(prompts)
        total = max((len(p) for p in prompts), default=0)
        pad = np.asarray([total - len(p) for p in prompts], dtype=np.int32)
        emb = np.zeros((b, total, self.cfg.hidden_size), dtype=self.precision.numpy_storage)
        for i, p in enumerate(prompts):
            if len(p):
                emb[i, pad[i]:] = self.embed(p)
        return self.generate_embeds(emb, pad, budget, eos, force_eot_step, chunk)

    def generate_embeds(self, embeds: np.ndarray, pad: Sequence[int], budget: int,
                        eos: int = DEFAULT_EOS, force_eot_step: Sequence[int] | None = None,
                        chunk: int = 256) -> list[Generated]:
        e = np.ascontiguousarray(embeds, dtype=self.precision.numpy_storage)
        b, t, _ = e.shape
        pad = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        tokens = np.zeros((b, budget), dtype=np.uint32)
        ntok = np.zeros(b, dtype=np.int32)
        fin = np.zeros(b, dtype=np.int32)
        force = None if force_eot_step is None else np.ascontiguousarray(
            np.asarray(force_eot_step, dtype=np.int32))
        _check(lib().fmd_dec_generate(self.handle, _ptr(e), 0, _ptr(pad), b, t, chunk, budget,
                                      eos, _ptr(force), _ptr(tokens), _ptr(ntok), _ptr(fin)))
        return [Generated(tokens[i, : ntok[i]].tolist(), FinishReason(int(fin[i])))
                for i in range(b)]

    def generate_device(self, embeds_dev, pad: Sequence[int], budget: int,
                        eos: int = DEFAULT_EOS, force_eot_step: Sequence[int] | None = None,
                        chunk: int = 256) -> list[Generated]:
        """generate_batch from a device (B, total, hidden) activation tensor,
        such as ``assemble`` returns, and its pads."""
        b, t, _ = embeds_dev.shape
        pad = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        tokens = np.zeros((b, budget), dtype=np.uint32)
        ntok = np.zeros(b, dtype=np.int32)
        fin = np.zeros(b, dtype=np.int32)
        force = None if force_eot_step is None else np.ascontiguousarray(
            np.asarray(force_eot_step, dtype=np.int32))
        _check(lib().fmd_dec_generate(self.handle, embeds_dev.data_ptr(), 1, _ptr(pad), b, t, chunk,
                                      budget, eos, _ptr(force), _ptr(tokens), _ptr(ntok), _ptr(fin)))
        return [Generated(tokens[i, : ntok[i]].tolist(), FinishReason(int(fin[i])))
                for i in range(b)]

    def decode_loop(self, caches: KvCache, first_ids: Sequence[int], pad: Sequence[int],
                    max_steps: int, eos: int = DEFAULT_EOS,
                    force_eot_step: Sequence[int] | None = None):
        """Greedy loop from an existing cache.  Returns (generated, steps_run)."""
        ids = np.ascontiguousarray(np.asarray(first_ids, dtype=np.uint32))
        b = ids.size
        pad = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        budget = max(max_steps, 1)
        tokens = np.zeros((b, budget), dtype=np.uint32)
        ntok = np.zeros(b, dtype=np.int32)
        fin = np.zeros(b, dtype=np.int32)
        steps = np.zeros(1, dtype=np.int32)
        force = None if force_eot_step is None else np.ascontiguousarray(
            np.asarray(force_eot_step, dtype=np.int32))
        _check(lib().fmd_dec_decode_loop(self.handle, caches.handle, _ptr(ids), _ptr(pad), b,
                                         max_steps, eos, _ptr(force), _ptr(tokens), _ptr(ntok),
                                         _ptr(fin), _ptr(steps)))
        gens = [Generated(tokens[i, : ntok[i]].tolist(), FinishReason(int(fin[i])))
                for i in range(b)]
        return gens, int(steps[0])

    def greedy(self, batch: int, step: int, done: np.ndarray, eos: int = DEFAULT_EOS,
               force_eot_step: Sequence[int] | None = None):
        """One greedy update (argmax_rows + engine.rs:505-531) on the device over
        the last prefill / decode_step logits.  `done` (int32, batch) is updated
        in place.  Returns (next_ids, emitted) with emitted[b] = -1 when row b
        emitted nothing this step."""
        assert done.dtype == np.int32 and done.flags.c_contiguous and done.size == batch
        nxt = np.zeros(batch, dtype=np.uint32)
        emitted = np.zeros(batch, dtype=np.uint32)
        force = None if force_eot_step is None else np.ascontiguousarray(
            np.asarray(force_eot_step, dtype=np.int32))
        _check(lib().fmd_dec_greedy(self.handle, batch, eos, _ptr(force), step, _ptr(done),
                                    _ptr(nxt), _ptr(emitted)))
        return nxt.tolist(), [int(v) if v != 0xFFFFFFFF else -1 for v in emitted]

    # -- device ops (tests / benchmarks) -------------------------------------
    def set_stream(self, stream_handle: int | None) -> None:
        _check(lib().fmd_dec_set_stream(self.handle, stream_handle))

    def op_attention_decode_noalloc(self, caches: KvCache, layer: int, qkv_ptr: int,
                                    pad: Sequence[int], batch: int, ctx_ptr: int) -> None:
        """op_attention_decode with its scratch in the library's static device
        array instead of allocated workspace (no allocation at all)."""
        p = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        _check(lib().fmd_op_attention_decode_noalloc(self.handle, caches.handle, layer, qkv_ptr,
                                                     _ptr(p), batch, ctx_ptr))

    def set_spin_limit(self, polls: int) -> None:
        """Polls before a wait of the decode attention gives up (the call then fails)."""
        _check(lib().fmd_dec_set_spin_limit(self.handle, polls))

    def op_layer_decode(self, caches: KvCache, layer: int, x_ptr: int, pad: Sequence[int],
                        batch: int) -> None:
        """One decoder layer for one new token per row, in place on the device
        rows at x_ptr (batch, hidden); the new K/V go to position caches.len(),
        which is not advanced."""
        p = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        _check(lib().fmd_op_layer_decode(self.handle, caches.handle, layer, x_ptr, _ptr(p), batch))

    def op_logits(self, x_ptr: int, rows: int, logits_ptr: int) -> None:
        """Final RMSNorm + lm_head of device rows x_ptr (rows, hidden) into f32
        device logits (rows, vocab)."""
        _check(lib().fmd_op_logits(self.handle, x_ptr, rows, logits_ptr))

    def op_linear(self, layer: int, proj: int, x_ptr: int, rows: int, y_ptr: int) -> None:
        _check(lib().fmd_op_linear(self.handle, layer, proj, x_ptr, rows, y_ptr))

    def op_attention_decode(self, caches: KvCache, layer: int, qkv_ptr: int,
                            pad: Sequence[int], batch: int, ctx_ptr: int) -> None:
        """Decode attention of one layer for the raw qkv projection (device
        pointer); the new K/V go to position caches.len(), which is not advanced."""
        p = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        _check(lib().fmd_op_attention_decode(self.handle, caches.handle, layer, qkv_ptr, _ptr(p),
                                             batch, ctx_ptr))


DEFAULT_GENERATION_MAX_NEW_TOKENS = 5120  # config.rs:103-106


@dataclass
class EngineConfig:
    """The decoder-relevant part of EngineConfig (engine.rs:70-96), plus what
    the engine takes from ``generation_config.json`` (engine.rs:246, 466-469):
    ``eos_id`` and the checkpoint's own cap ``generation_max_new_tokens``.
    ``checkpoint.engine_config`` fills both from a checkpoint directory."""

    max_new_tokens: int = 4096
    max_batch_size: int = 8
    eos_id: int = DEFAULT_EOS
    chunk: int = 256
    generation_max_new_tokens: int = DEFAULT_GENERATION_MAX_NEW_TOKENS

    def budget(self) -> int:
        """Tokens per request: min(max_new_tokens, max(generation cap, 1))
        (engine.rs:466-469)."""
        return min(int(self.max_new_tokens), max(int(self.generation_max_new_tokens), 1))


@dataclass
class Result:
    tokens: list[int]
    finish_reason: FinishReason
    prompt_tokens: int
    error: str | None = None


class Engine:
    """Length-sorted micro-batching over token-id prompts (engine.rs:382-428)."""

    def __init__(self, model: Qwen3, cfg: EngineConfig | None = None):
        self.model = model
        self.cfg = cfg or EngineConfig()

    def generate(self, prompts: Sequence[Sequence[int]],
                 force_eot_step: Sequence[int] | None = None) -> tuple[list[Result], BatchStats]:
        n = len(prompts)
        lens = np.asarray([len(p) for p in prompts], dtype=np.int64)
        ids = np.ascontiguousarray(
            np.concatenate([np.asarray(p, dtype=np.uint32) for p in prompts])
            if n and lens.sum() else np.zeros(1, dtype=np.uint32))
        budget = self.cfg.budget()
        tokens = np.zeros((max(n, 1), budget), dtype=np.uint32)
        ntok = np.zeros(max(n, 1), dtype=np.int32)
        fin = np.zeros(max(n, 1), dtype=np.int32)
        status = np.zeros(max(n, 1), dtype=np.int32)
        force = None if force_eot_step is None else np.ascontiguousarray(
            np.asarray(force_eot_step, dtype=np.int32))
        stats = BatchStats()
        stride = 512
        errors = ctypes.create_string_buffer(max(n, 1) * stride)
        _check(lib().fmd_engine_generate(self.model.handle, _ptr(ids), _ptr(lens), n,
                                         self.cfg.max_batch_size, budget, self.cfg.eos_id,
                                         _ptr(force), self.cfg.chunk, _ptr(tokens), _ptr(ntok),
                                         _ptr(fin), _ptr(status), errors, stride,
                                         ctypes.byref(stats)))
        out = []
        for i in range(n):
            # "batch generation failed: {e}" for every member of a failed
            # micro-batch (engine.rs:414-421)
            err = None if status[i] == 0 else (
                errors.raw[i * stride:(i + 1) * stride].split(b"\0", 1)[0].decode())
            out.append(Result(tokens[i, : ntok[i]].tolist(), FinishReason(int(fin[i])),
                              int(lens[i]), err))
        return out, stats
