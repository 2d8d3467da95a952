"""``transcribe_batch`` over encoded requests: prompt ids and audio
embeddings in, diarised transcripts out, on the HIP decoder.

It follows ``Engine::transcribe`` (engine.rs:285-428) from the splice on,
and the Python binding's ``transcribe_batch`` (fmd-py lib.rs:270-298):

1. Each request's prompt must hold one audio placeholder per audio row
   (``splice_audio``, mod.rs:137-150); a request that does not fails alone
   with the reference's message and the others go on (engine.rs:359-380).
2. The requests left are sorted by prompt length (a stable sort) and cut into
   micro-batches of ``max(max_batch_size, 1)`` (engine.rs:383-387).
3. Each micro-batch is assembled on the device -- token embeddings, audio
   rows spliced into the placeholders, left padding (``fmd_dec_assemble``) --
   and generated greedily (``fmd_dec_generate``).  A failure fails every
   member with ``batch generation failed: {e}`` (engine.rs:414-421).
4. Each output is decoded without special tokens, trimmed, and parsed into
   segments (engine.rs:393-412, prompt.rs:153-155, transcript.rs:21-58).

A request carries the encoder's output rows (``EncodedRequest``), or its
log-mel chunks (``MelRequest``): ``transcribe_mel`` first runs every chunk of
every request through the HIP encoder and adaptor in one batched pass
(``MossModel::encode_audio``, engine.rs:329-346, mod.rs:82-126) and then
continues as above.  The audio decode and log-mel front end stay on the
reference path.  With ``raise_on_error`` (the default, as in the binding) the
first failed slot raises; otherwise it holds a ``Failure``.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import transcript
from .decoder import EngineConfig, FinishReason, FmdError, Qwen3


@dataclass
class EncodedRequest:
    """One request after prompt rendering and audio encoding."""

    id: str
    prompt_ids: Sequence[int]
    audio: object = None          # (rows, hidden) numpy or torch, f32 / f16 / bf16; None: no audio
    audio_seconds: float = 0.0


@dataclass
class MelRequest:
    """One request before audio encoding: its log-mel chunks (n_chunks,
    n_mels, frames) as the front end cuts them (30 s each, the last one
    padded), the encoder tokens each chunk contributes
    (``chunk_token_lengths``, audio/mod.rs), and prompt ids already holding
    one audio placeholder per token (PromptBuilder::build, prompt.rs)."""

    id: str
    prompt_ids: Sequence[int]
    mel: object
    chunk_tokens: Sequence[int]
    audio_seconds: float = 0.0


@dataclass
class Response:
    """engine.rs:141-149."""

    id: str
    text: str
    segments: list
    prompt_tokens: int
    generated_tokens: int
    audio_seconds: float
    finish_reason: FinishReason


@dataclass
class Failure:
    """A failed slot (the binding's ``Failure``): the request id and the error text."""

    id: str
    error: str


@dataclass
class TranscribeStats:
    """The decoder-side part of BatchStats (engine.rs:151-174)."""

    requests: int = 0
    encode_seconds: float = 0.0
    generate_seconds: float = 0.0
    audio_seconds: float = 0.0
    generated_tokens: int = 0
    micro_batches: int = 0


def _audio_rows(audio) -> int:
    return 0 if audio is None else int(audio.shape[0])


def build_response(req: EncodedRequest, tokens: Sequence[int], finish: FinishReason,
                   tokenizer) -> Response:
    """Decode, trim and parse one generated sequence (engine.rs:393-412)."""
    text = transcript._trim(transcript.decode(tokenizer, tokens))
    return Response(id=req.id, text=text, segments=transcript.parse(text),
                    prompt_tokens=len(req.prompt_ids), generated_tokens=len(tokens),
                    audio_seconds=req.audio_seconds, finish_reason=finish)


@dataclass
class Transcriber:
    """A decoder, its tokenizer (``tokenizers.Tokenizer`` or the path of a
    ``tokenizer.json``) and the engine options."""

    model: Qwen3
    tokenizer: object
    audio_token_id: int
    cfg: EngineConfig = field(default_factory=EngineConfig)
    encoder: object = None        # AudioEncoder, for transcribe_mel
    encoder_batch: int = 16       # EngineConfig::encoder_batch (engine.rs:70-96)

    def __post_init__(self):
        if isinstance(self.tokenizer, str) or hasattr(self.tokenizer, "__fspath__"):
            from tokenizers import Tokenizer

            self.tokenizer = Tokenizer.from_file(str(self.tokenizer))

    def transcribe_batch(self, requests: Sequence[EncodedRequest], *, raise_on_error: bool = True,
                         force_eot_step: Sequence[int] | None = None):
        """(results in request order, stats).  ``force_eot_step`` (per request,
        optional) replaces a row's argmax by end-of-turn at that greedy step."""
        n = len(requests)
        results: list = [None] * n
        stats = TranscribeStats(requests=n)
        stats.audio_seconds = float(sum(r.audio_seconds for r in requests))
        pending = []
        for slot, req in enumerate(requests):
            ids = [int(t) for t in req.prompt_ids]
            slots = sum(1 for t in ids if t == self.audio_token_id)
            rows = _audio_rows(req.audio)
            if slots != rows:  # mod.rs:145-150
                results[slot] = Failure(req.id, f"prompt has {slots} audio placeholders but the "
                                                f"encoder produced {rows} embeddings")
            else:
                pending.append(slot)
        t0 = time.perf_counter()
        pending.sort(key=lambda s: len(requests[s].prompt_ids))  # stable (engine.rs:385)
        step = max(int(self.cfg.max_batch_size), 1)
        for g0 in range(0, len(pending), step):
            group = pending[g0:g0 + step]
            stats.micro_batches += 1
            try:
                embeds, pad = self.model.assemble(
                    [requests[s].prompt_ids for s in group],
                    audio=[requests[s].audio for s in group],
                    audio_token_id=self.audio_token_id)
                force = None if force_eot_step is None else [force_eot_step[s] for s in group]
                outs = self.model.generate_device(embeds, pad, self.cfg.budget(),
                                                  eos=self.cfg.eos_id, force_eot_step=force,
                                                  chunk=self.cfg.chunk)
            except FmdError as e:
                for s in group:
                    results[s] = Failure(requests[s].id, f"batch generation failed: {e}")
                continue
            for s, out in zip(group, outs):
                stats.generated_tokens += len(out.tokens)
                try:
                    results[s] = build_response(requests[s], out.tokens, out.finish_reason,
                                                self.tokenizer)
                except Exception as e:  # a tokenizer error fails that request alone
                    results[s] = Failure(requests[s].id, str(e))
        stats.generate_seconds = time.perf_counter() - t0
        if raise_on_error:  # fmd-py lib.rs:376-377: "{id}: {e}"
            for r in results:
                if isinstance(r, Failure):
                    raise FmdError(-1, f"{r.id}: {r.error}")
        return results, stats

    def transcribe_mel(self, requests: Sequence[MelRequest], *, raise_on_error: bool = True,
                       force_eot_step: Sequence[int] | None = None):
        """``transcribe_batch`` from log-mel chunks: one batched encoder pass
        over every chunk of every request (chunk i of the stack belongs to its
        request, engine.rs:329-346; an encoder failure fails the whole call, as
        the reference's ``?`` does), then splice, sort, generate and parse."""
        if self.encoder is None:
            raise FmdError(-2, "transcribe_mel needs an AudioEncoder")
        mels, tokens, mapping = [], [], []
        for i, r in enumerate(requests):
            m = np.asarray(r.mel, dtype=np.float32)
            if m.ndim != 3 or m.shape[0] != len(r.chunk_tokens):
                raise FmdError(-1, f"{r.id}: mel must be (n_chunks, n_mels, frames) with one "
                                   f"token length per chunk")
            mels.append(m)
            tokens.extend(int(t) for t in r.chunk_tokens)
            mapping.extend([i] * m.shape[0])
        t0 = time.perf_counter()
        if mels and sum(m.shape[0] for m in mels):
            audio = self.encoder.encode_audio(np.concatenate(mels), tokens, mapping, len(requests),
                                              encoder_batch=self.encoder_batch)
        else:
            audio = [None] * len(requests)
        encode_seconds = time.perf_counter() - t0
        enc = [EncodedRequest(r.id, r.prompt_ids, a if a is not None and a.shape[0] else None,
                              r.audio_seconds) for r, a in zip(requests, audio)]
        results, stats = self.transcribe_batch(enc, raise_on_error=raise_on_error,
                                               force_eot_step=force_eot_step)
        stats.encode_seconds = encode_seconds
        return results, stats
