"""Local checkpoint ingest: a MOSS-Transcribe-Diarize directory -> Qwen3 decoder.

Follows the reference's local model source and loader:

* ``resolve_local`` (hub.rs:88-133): every ``*.safetensors`` file of the
  directory, sorted by path, and a required ``config.json``.  The tokenizer
  and preprocessor files the full pipeline also requires are not needed by the
  decoder and are not checked here.
* ``ModelConfig.text_config`` (config.rs:8-41, 77-91) with the serde defaults.
* ``Qwen3::load`` names (qwen3.rs:354-390): everything under
  ``model.language_model.``; the output projection from
  ``model.language_model.lm_head.weight``, else a root ``lm_head.weight``,
  else tied to the embedding (qwen3.rs:566-578).  Other tensors (the Whisper
  encoder and the adaptor) belong to the reference path and are skipped.
* Loader precision views (linear.rs:102-153): tensors go to the device in
  their stored dtype; the decoder rounds them to the activation dtype, and in
  int8 quantises projections from the exact f32 widening of the stored values.
* ``generation_config.json`` (optional, hub.rs:125; config.rs:91-117): the
  end-of-turn id (``eos_token_id``, else 151645, engine.rs:246) and the
  checkpoint's token cap (``max_new_tokens``, default 5120), which bounds the
  engine's budget (engine.rs:466-469).

Tensors are read with safetensors' own loader (no pickled code is executed),
one at a time, so host memory holds one tensor beyond the mapping.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

from .decoder import (DEFAULT_EOS, DEFAULT_GENERATION_MAX_NEW_TOKENS, EngineConfig, FmdError,
                      Precision, Qwen3, TextConfig)

PREFIX = "model.language_model."
_TEXT_FIELDS = (
    "vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
    "num_attention_heads", "num_key_value_heads",
)


class CheckpointError(FmdError):
    """A checkpoint directory the decoder cannot load (hub.rs:88-133 errors)."""

    def __init__(self, message: str):
        super().__init__(-1, message)


def resolve_local(directory: str | Path) -> tuple[Path, list[Path]]:
    """(config.json, sorted *.safetensors) of a local checkpoint (hub.rs:88-133)."""
    d = Path(directory)
    if not d.is_dir():
        raise CheckpointError(f"{d} is not a directory")
    weights = sorted(p for p in d.iterdir() if p.suffix == ".safetensors" and p.is_file())
    if not weights:
        raise CheckpointError(f"no .safetensors weights found in {d}")
    config = d / "config.json"
    if not config.is_file():
        raise CheckpointError(f"config.json is missing from the checkpoint at {d}")
    return config, weights


def text_config(config_json: str | Path | dict) -> TextConfig:
    """``text_config`` of a top-level config.json, with config.rs's defaults."""
    raw = config_json if isinstance(config_json, dict) else json.loads(Path(config_json).read_text())
    tc = raw.get("text_config")
    if not isinstance(tc, dict):
        raise CheckpointError("config.json has no text_config")
    missing = [k for k in _TEXT_FIELDS if k not in tc]
    if missing:
        raise CheckpointError(f"text_config is missing {', '.join(missing)}")
    kw = {k: int(tc[k]) for k in _TEXT_FIELDS}
    kw["head_dim"] = int(tc.get("head_dim", 128))
    kw["rms_norm_eps"] = float(tc.get("rms_norm_eps", 1e-6))
    kw["rope_theta"] = float(tc.get("rope_theta", 1_000_000.0))
    kw["max_position_embeddings"] = int(tc.get("max_position_embeddings", 131_072))
    kw["tie_word_embeddings"] = bool(tc.get("tie_word_embeddings", False))
    kw["attention_bias"] = bool(tc.get("attention_bias", False))
    return TextConfig(**kw)


def decoder_tensor(name: str) -> bool:
    """Whether a checkpoint tensor belongs to the decoder (qwen3.rs:354-390)."""
    return name.startswith(PREFIX) or name == "lm_head.weight"


def load_into(model, weights: list[Path]) -> int:
    """Stream every decoder tensor of the files into ``model.set_weight``.

    An output projection under the prefix wins over a root ``lm_head.weight``
    (the reference looks for it first), so the root one is applied only when
    the prefixed one is absent.  Returns the number of tensors loaded."""
    import torch
    from safetensors import safe_open

    names: dict[str, Path] = {}
    for f in weights:
        with safe_open(str(f), framework="pt", device="cpu") as fh:
            for n in fh.keys():
                if decoder_tensor(n):
                    if n in names:
                        raise CheckpointError(f"tensor {n} appears in {names[n].name} and {f.name}")
                    names[n] = f
    if PREFIX + "lm_head.weight" in names:
        names.pop("lm_head.weight", None)
    count = 0
    for f in weights:
        mine = [n for n, g in names.items() if g == f]
        if not mine:
            continue
        with safe_open(str(f), framework="pt", device="cpu") as fh:
            for n in mine:
                t = fh.get_tensor(n)
                if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
                    t = t.to(torch.float32)
                model.set_weight(n, t)
                count += 1
    return count


def load_checkpoint(directory: str | Path, precision: Precision | str = Precision.BF16,
                    device: int = 0, max_len: int | None = None) -> Qwen3:
    """The decoder of a local checkpoint directory, ready to run."""
    config, weights = resolve_local(directory)
    model = Qwen3(text_config(config), precision, device=device, max_len=max_len)
    load_into(model, weights)
    if not model.ready():
        raise CheckpointError(f"the checkpoint at {directory} lacks decoder weights")
    return model


@dataclass
class GenerationConfig:
    """``generation_config.json`` (config.rs:91-117).  Absent file: the
    reference's ``Default`` (ids 151643 / 151645 / 151643, 5120 tokens);
    a field absent from a present file: ``None`` ids, 5120 tokens."""

    bos_token_id: int | None = 151_643
    eos_token_id: int | None = DEFAULT_EOS
    pad_token_id: int | None = 151_643
    max_new_tokens: int = DEFAULT_GENERATION_MAX_NEW_TOKENS


def _opt_id(raw: dict, key: str) -> int | None:
    v = raw.get(key)
    if v is None:
        return None
    if isinstance(v, bool) or not isinstance(v, int) or v < 0 or v > 0xFFFFFFFF:
        raise CheckpointError(f"generation_config.json: {key} must be an unsigned 32-bit id")
    return int(v)


def generation_config(directory: str | Path) -> GenerationConfig:
    """The checkpoint's generation settings (engine.rs:225-232)."""
    p = Path(directory) / "generation_config.json"
    if not p.is_file():
        return GenerationConfig()
    try:
        raw = json.loads(p.read_text())
    except json.JSONDecodeError as e:
        raise CheckpointError(f"generation_config.json: {e}") from None
    if not isinstance(raw, dict):
        raise CheckpointError("generation_config.json: expected an object")
    mnt = raw.get("max_new_tokens", DEFAULT_GENERATION_MAX_NEW_TOKENS)
    if isinstance(mnt, bool) or not isinstance(mnt, int) or mnt < 0:
        raise CheckpointError("generation_config.json: max_new_tokens must be a non-negative integer")
    return GenerationConfig(bos_token_id=_opt_id(raw, "bos_token_id"),
                            eos_token_id=_opt_id(raw, "eos_token_id"),
                            pad_token_id=_opt_id(raw, "pad_token_id"),
                            max_new_tokens=int(mnt))


def engine_config(directory: str | Path, max_new_tokens: int = 4096, max_batch_size: int = 8,
                  chunk: int = 256) -> EngineConfig:
    """Engine options for a checkpoint: eos = generation.eos_token_id, else
    151645 (engine.rs:246); the per-request budget is min(max_new_tokens,
    max(generation.max_new_tokens, 1)) (engine.rs:466-469)."""
    g = generation_config(directory)
    return EngineConfig(max_new_tokens=max_new_tokens, max_batch_size=max_batch_size,
                        eos_id=DEFAULT_EOS if g.eos_token_id is None else g.eos_token_id,
                        chunk=chunk, generation_max_new_tokens=g.max_new_tokens)
