"""ctypes wrapper over liboracle.so -- the CPU restatement of the reference
decoder (fmd_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker used by tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg.  The product never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# FMD_ORACLE_LIB selects another build of the same sources (the sanitizer
# build of tests/test_sanitized.py).
LIB = Path(os.environ.get("FMD_ORACLE_LIB") or HERE / "liboracle.so")

F32, F16, BF16, INT8 = 0, 1, 2, 3
PREC = {"f32": F32, "fp32": F32, "f16": F16, "fp16": F16, "bf16": BF16, "int8": INT8}


class Cfg(ctypes.Structure):
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


class AudioCfg(ctypes.Structure):
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


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        h = ctypes.CDLL(str(LIB))
        sig = {
            "or_f32_to_f16": (ctypes.c_uint16, [_F]),
            "or_f16_to_f32": (_F, [ctypes.c_uint16]),
            "or_f32_to_bf16": (ctypes.c_uint16, [_F]),
            "or_bf16_to_f32": (_F, [ctypes.c_uint16]),
            "or_round": (_F, [_F, _I]),
            "or_round_array": (None, [_P, _I64, _I]),
            "or_quantize_q8_0": (None, [_P, _I64, _I64, _P]),
            "or_dequantize_q8_0": (None, [_P, _I64, _I64, _P]),
            "or_rope_tables": (None, [_I, ctypes.c_double, _I, _I, _P, _P]),
            "or_build_mask": (None, [_I, _I, _I, _I, _I, _P, _P]),
            "or_rope_apply": (None, [_P, _I, _I, _I, _I, _I, _P, _P, _I]),
            "or_rmsnorm": (None, [_P, _P, _I64, _I, _F, _I, _P]),
            "or_linear_dense": (None, [_P, _P, _I64, _I, _I, _I, _P]),
            "or_linear_q8_0": (None, [_P, _P, _I64, _I, _I, _I, _P]),
            "or_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
            "or_model_new": (_P, [ctypes.POINTER(Cfg), _I, _I]),
            "or_model_free": (None, [_P]),
            "or_model_set": (_I, [_P, ctypes.c_char_p, _P]),
            "or_model_ready": (_I, [_P]),
            "or_model_fill_random": (_I, [_P, ctypes.c_uint64, _F]),
            "or_last_error": (ctypes.c_char_p, []),
            "or_kv_new": (_P, [_P, _I, _I]),
            "or_kv_free": (None, [_P]),
            "or_kv_len": (_I, [_P]),
            "or_kv_read": (_I, [_P, _I, _I, _P]),
            "or_kv_write": (_I, [_P, _I, _I, _P]),
            "or_kv_set_len": (_I, [_P, _I]),
            "or_kv_fill_random": (_I, [_P, ctypes.c_uint64, _I, _I]),
            "or_embed": (None, [_P, _P, _I64, _P]),
            "or_prefill": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
            "or_decode_step": (_I, [_P, _P, _P, _P, _I, _P]),
            "or_argmax_rows": (None, [_P, _I, _I, _P]),
            "or_layer_decode": (_I, [_P, _P, _I, _P, _P, _I]),
            "or_final_logits": (None, [_P, _P, _I, _P]),
            "or_generate": (_I, [_P, _P, _P, _I, _I, _I, _I, ctypes.c_uint32, _P, _P, _P, _P]),
            "or_set_threads": (None, [_I]),
            "or_conv1d": (None, [_P, _P, _I, _I, _I, _I, _I, _I, _P]),
            "or_gelu_erf": (None, [_P, _I64, _I]),
            "or_silu": (None, [_P, _I64, _I]),
            "or_layernorm": (None, [_P, _P, _P, _I64, _I, _F, _I, _P]),
            "or_attention_dense": (None, [_P, _P, _P, _I, _I, _I, _I, _P]),
            "or_enc_new": (_P, [ctypes.POINTER(AudioCfg), _I]),
            "or_enc_free": (None, [_P]),
            "or_enc_set": (_I, [_P, ctypes.c_char_p, _P]),
            "or_enc_ready": (_I, [_P]),
            "or_enc_last_error": (ctypes.c_char_p, []),
            "or_enc_stem": (_I, [_P, _P, _I, _I, _P]),
            "or_enc_layers": (_I, [_P, _P, _I, _I, _I, _I, _I]),
            "or_enc_forward": (_I, [_P, _P, _I, _I, _P]),
            "or_enc_adaptor": (_I, [_P, _P, _I, _P]),
            "or_enc_encode_audio": (_I, [_P, _P, _I, _I, _P, _P, _I, _P, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


class OracleError(RuntimeError):
    pass


def _ck(rc):
    if rc != 0:
        raise OracleError(lib().or_last_error().decode())


# ---- conversions -----------------------------------------------------------

def round_to(x: np.ndarray, prec: int) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().or_round_array(_p(a), a.size, prec)
    return a


def to_storage(x: np.ndarray, prec: int) -> np.ndarray:
    """f32 values -> storage of the activation dtype (f32, f16, or bf16 bits)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    if prec == F32:
        return a.copy()
    if prec in (F16, INT8):
        return round_to(a, F16).astype(np.float16)
    r = round_to(a, BF16)
    return (r.view(np.uint32) >> 16).astype(np.uint16)


def from_storage(a: np.ndarray, prec: int) -> np.ndarray:
    if prec == BF16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.empty((rows, cols // 32, 34), dtype=np.uint8)
    lib().or_quantize_q8_0(_p(x), rows, cols, _p(out))
    return out


def dequantize_q8_0(blocks: np.ndarray, rows: int, cols: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty((rows, cols), dtype=np.float32)
    lib().or_dequantize_q8_0(_p(b), rows, cols, _p(out))
    return out


def rope_tables(head_dim: int, theta: float, max_len: int, prec: int):
    c = np.empty((max_len, head_dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    lib().or_rope_tables(head_dim, theta, max_len, prec, _p(c), _p(s))
    return c, s


def rope_apply(x, offset, cos_t, sin_t, prec=F32):
    """x (b, heads, t, hd) -> rotated copy at absolute `offset`."""
    a = np.ascontiguousarray(x, dtype=np.float32).copy()
    b, h, t, hd = a.shape
    c = np.ascontiguousarray(cos_t, dtype=np.float32)
    s = np.ascontiguousarray(sin_t, dtype=np.float32)
    lib().or_rope_apply(_p(a), b, h, t, hd, offset, _p(c), _p(s), prec)
    return a


def build_mask(batch, repeat, q_offset, q_len, kv_len, pad):
    pad = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
    out = np.empty((batch, 1, repeat * q_len, kv_len), dtype=np.float32)
    lib().or_build_mask(batch, repeat, q_offset, q_len, kv_len, _p(pad), _p(out))
    return out


def rmsnorm(x, w, eps, prec=F32):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty_like(x)
    dim = x.shape[-1]
    lib().or_rmsnorm(_p(x), _p(w), x.size // dim, dim, eps, prec, _p(y))
    return y


def linear_dense(x, w, prec=F32):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows = x.size // x.shape[-1]
    y = np.empty(x.shape[:-1] + (w.shape[0],), dtype=np.float32)
    lib().or_linear_dense(_p(x), _p(w), rows, w.shape[1], w.shape[0], prec, _p(y))
    return y


def linear_q8_0(x, blocks, out_dim, prec=F16):
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = x.size // x.shape[-1]
    y = np.empty(x.shape[:-1] + (out_dim,), dtype=np.float32)
    lib().or_linear_q8_0(_p(x), _p(b), rows, x.shape[-1], out_dim, prec, _p(y))
    return y


def attention(q, k, v, mask, kv_len, prec=F32):
    """q (b, heads, t, hd); k, v (b, kvh, stride, hd); mask (b,1,rep*t,kv_len) or None."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    b, heads, t, hd = q.shape
    kvh, stride = k.shape[1], k.shape[2]
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
    out = np.empty((b, t, heads * hd), dtype=np.float32)
    lib().or_attention(_p(q), _p(k), _p(v), _p(m), b, heads, kvh, t, kv_len, stride, hd, prec,
                       _p(out))
    return out


def argmax_rows(logits):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty(l.shape[0], dtype=np.uint32)
    lib().or_argmax_rows(_p(l), l.shape[0], l.shape[1], _p(out))
    return out


# ---- model -------------------------------------------------------------------

def cfg_c(cfg) -> Cfg:
    return Cfg(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers,
               cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
               cfg.max_position_embeddings, float(cfg.rms_norm_eps), float(cfg.rope_theta),
               int(getattr(cfg, "tie_word_embeddings", True)), int(getattr(cfg, "attention_bias", False)))


class OracleKv:
    def __init__(self, model: "OracleModel", batch: int, capacity: int):
        self.model = model
        self.batch = batch
        self.capacity = capacity
        self.h = lib().or_kv_new(model.h, batch, capacity)
        if not self.h:
            raise OracleError(lib().or_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_kv_free(self.h)
            self.h = None

    def len(self) -> int:
        return lib().or_kv_len(self.h)

    def shape(self):
        c = self.model.cfg
        return (self.batch, c.num_key_value_heads, self.capacity, c.head_dim)

    def read(self, layer, which) -> np.ndarray:
        out = np.empty(self.shape(), dtype=np.float32)
        _ck(lib().or_kv_read(self.h, layer, which, _p(out)))
        return out

    def write(self, layer, which, data):
        d = np.ascontiguousarray(data, dtype=np.float32)
        _ck(lib().or_kv_write(self.h, layer, which, _p(d)))

    def set_len(self, n):
        _ck(lib().or_kv_set_len(self.h, n))

    def fill_random(self, seed, n):
        _ck(lib().or_kv_fill_random(self.h, seed, n, self.model.prec))


class OracleModel:
    def __init__(self, cfg, prec: int, max_len: int):
        self.cfg = cfg
        self.prec = prec
        self.max_len = max_len
        c = cfg_c(cfg)
        self.h = lib().or_model_new(ctypes.byref(c), prec, max_len)
        if not self.h:
            raise OracleError(lib().or_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None

    def load(self, weights: dict) -> "OracleModel":
        for name, w in weights.items():
            a = np.ascontiguousarray(w, dtype=np.float32)
            _ck(lib().or_model_set(self.h, name.encode(), _p(a)))
        assert lib().or_model_ready(self.h)
        return self

    def fill_random(self, seed: int, std: float = 0.02) -> "OracleModel":
        _ck(lib().or_model_fill_random(self.h, seed, std))
        return self

    def new_kv(self, batch, capacity) -> OracleKv:
        return OracleKv(self, batch, capacity)

    def embed(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32).reshape(-1))
        out = np.empty((ids.size, self.cfg.hidden_size), dtype=np.float32)
        lib().or_embed(self.h, _p(ids), ids.size, _p(out))
        return out

    def prefill(self, kv: OracleKv, embeds, pad, block=256) -> np.ndarray:
        e = np.ascontiguousarray(embeds, dtype=np.float32)
        b, t, _ = e.shape
        pad = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        logits = np.empty((b, self.cfg.vocab_size), dtype=np.float32)
        _ck(lib().or_prefill(self.h, kv.h, _p(e), _p(pad), b, t, block, _p(logits)))
        return logits

    def decode_step(self, kv: OracleKv, ids, pad) -> np.ndarray:
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
        pad = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        logits = np.empty((ids.size, self.cfg.vocab_size), dtype=np.float32)
        _ck(lib().or_decode_step(self.h, kv.h, _p(ids), _p(pad), ids.size, _p(logits)))
        return logits

    def layer_decode(self, kv: OracleKv, layer: int, x, pad) -> np.ndarray:
        """One decoder layer for one new token per row at kv.len() (not advanced)."""
        out = np.ascontiguousarray(x, dtype=np.float32).copy()
        pad = np.ascontiguousarray(np.asarray(pad, dtype=np.int32))
        _ck(lib().or_layer_decode(self.h, kv.h, layer, _p(out), _p(pad), out.shape[0]))
        return out

    def final_logits(self, x) -> np.ndarray:
        """Final RMSNorm + lm_head of rows x (rows, hidden)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty((x.shape[0], self.cfg.vocab_size), dtype=np.float32)
        lib().or_final_logits(self.h, _p(x), x.shape[0], _p(out))
        return out

    def padded_embeds(self, prompts):
        total = max(len(p) for p in prompts)
        pad = np.asarray([total - len(p) for p in prompts], dtype=np.int32)
        emb = np.zeros((len(prompts), total, self.cfg.hidden_size), dtype=np.float32)
        for i, p in enumerate(prompts):
            if len(p):
                emb[i, pad[i]:] = self.embed(p)
        return emb, pad

    def generate(self, prompts, budget, eos, force=None, block=256):
        emb, pad = self.padded_embeds(prompts)
        b, t, _ = emb.shape
        tokens = np.zeros((b, budget), dtype=np.uint32)
        ntok = np.zeros(b, dtype=np.int32)
        fin = np.zeros(b, dtype=np.int32)
        f = None if force is None else np.ascontiguousarray(np.asarray(force, dtype=np.int32))
        _ck(lib().or_generate(self.h, _p(emb), _p(pad), b, t, block, budget, eos, _p(f),
                              _p(tokens), _p(ntok), _p(fin)))
        return [(tokens[i, : ntok[i]].tolist(), int(fin[i])) for i in range(b)]


def set_threads(n: int) -> None:
    lib().or_set_threads(n)


# ---- audio path (fmd_oracle_encoder.c) ---------------------------------------

def conv1d(x, w, stride, prec=F32):
    """x (b, cin, t), w (cout, cin, 3), padding 1 -> (b, cout, tout) rounded."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b, cin, t = x.shape
    cout = w.shape[0]
    tout = (t + 2 - 3) // stride + 1
    out = np.empty((b, cout, tout), dtype=np.float32)
    lib().or_conv1d(_p(x), _p(w), b, cin, cout, t, stride, prec, _p(out))
    return out


def gelu_erf(x, prec=F32):
    a = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().or_gelu_erf(_p(a), a.size, prec)
    return a


def silu(x, prec=F32):
    a = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().or_silu(_p(a), a.size, prec)
    return a


def layernorm(x, w, b, eps, prec=F32):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    y = np.empty_like(x)
    dim = x.shape[-1]
    lib().or_layernorm(_p(x), _p(w), _p(b), x.size // dim, dim, eps, prec, _p(y))
    return y


def attention_dense(q, k, v, heads, prec=F32):
    """q, k, v (t, heads*hd) of one window -> (t, heads*hd)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    t, d = q.shape
    out = np.empty_like(q)
    lib().or_attention_dense(_p(q), _p(k), _p(v), t, heads, d // heads, prec, _p(out))
    return out


def audio_cfg_c(cfg) -> AudioCfg:
    return AudioCfg(cfg.num_mel_bins, cfg.d_model, cfg.encoder_layers,
                    cfg.encoder_attention_heads, cfg.encoder_ffn_dim, cfg.max_source_positions,
                    cfg.adaptor_input_dim, cfg.hidden_size, cfg.audio_merge_size,
                    float(cfg.norm_eps))


def _eck(rc):
    if rc != 0:
        raise OracleError(lib().or_enc_last_error().decode())


class OracleEncoder:
    """Whisper encoder + VqAdaptor (whisper_encoder.rs, adaptor.rs, mod.rs:82-126)."""

    def __init__(self, cfg, prec: int):
        self.cfg = cfg
        self.prec = prec
        c = audio_cfg_c(cfg)
        self.h = lib().or_enc_new(ctypes.byref(c), prec)
        if not self.h:
            raise OracleError(lib().or_enc_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_enc_free(self.h)
            self.h = None

    def load(self, weights: dict) -> "OracleEncoder":
        for name, w in weights.items():
            a = np.ascontiguousarray(w, dtype=np.float32)
            _eck(lib().or_enc_set(self.h, name.encode(), _p(a)))
        assert lib().or_enc_ready(self.h), "incomplete audio weights"
        return self

    def out_frames(self, frames: int) -> int:
        return (frames + 2 - 3) // 2 + 1

    def stem(self, mel) -> np.ndarray:
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        b, _, frames = mel.shape
        out = np.empty((b, self.out_frames(frames), self.cfg.d_model), dtype=np.float32)
        _eck(lib().or_enc_stem(self.h, _p(mel), b, frames, _p(out)))
        return out

    def layers(self, x, first: int, n: int, final_norm: bool = False) -> np.ndarray:
        out = np.ascontiguousarray(x, dtype=np.float32).copy()
        w, t, _ = out.shape
        _eck(lib().or_enc_layers(self.h, _p(out), w, t, first, n, int(final_norm)))
        return out

    def forward(self, mel) -> np.ndarray:
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        b, _, frames = mel.shape
        out = np.empty((b, self.out_frames(frames), self.cfg.d_model), dtype=np.float32)
        _eck(lib().or_enc_forward(self.h, _p(mel), b, frames, _p(out)))
        return out

    def adaptor(self, frames) -> np.ndarray:
        f = np.ascontiguousarray(frames, dtype=np.float32)
        g = f.shape[0] // self.cfg.audio_merge_size
        out = np.empty((g, self.cfg.hidden_size), dtype=np.float32)
        _eck(lib().or_enc_adaptor(self.h, _p(f), f.shape[0], _p(out)))
        return out

    def encode_audio(self, mel, chunk_tokens, chunk_mapping, num_audios):
        """Per-audio embeddings (list of (tokens, hidden) arrays)."""
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        n, _, frames = mel.shape
        ct = np.ascontiguousarray(np.asarray(chunk_tokens, dtype=np.int32))
        cm = np.ascontiguousarray(np.asarray(chunk_mapping, dtype=np.int32))
        t2 = self.out_frames(frames)
        total = int(sum(min(int(k) * self.cfg.audio_merge_size, t2) for k in ct))
        out = np.empty((max(total // self.cfg.audio_merge_size, 1), self.cfg.hidden_size),
                       dtype=np.float32)
        offs = np.zeros(num_audios + 1, dtype=np.int64)
        _eck(lib().or_enc_encode_audio(self.h, _p(mel), n, frames, _p(ct), _p(cm), num_audios,
                                       _p(out), _p(offs)))
        return [out[offs[a]:offs[a + 1]] for a in range(num_audios)]
