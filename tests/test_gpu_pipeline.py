"""The transcribe_batch facade on the device: encoded requests (prompt ids
with audio placeholders + audio rows) through device assembly, batched greedy
generation, decode and parse.  Each response's tokens equal generate_batch on
the same micro-batch assembled on the host (a numpy restatement of
splice_audio + left pad, mod.rs:128-180, engine.rs:476-491); its text is the
tokenizer's decode of them, trimmed, and its segments are parse(text).  A
request with a placeholder/row mismatch fails alone; a micro-batch whose rows
run past the RoPE table fails every member."""
import numpy as np
import pytest
import torch

from tests.gpu_util import tiny_cfg

pytestmark = pytest.mark.gpu

AUDIO = 1000
EOS = 1001


def _tokenizer(vocab_size):
    from tokenizers import Tokenizer, models, pre_tokenizers

    vocab = {f"w{i}": i for i in range(vocab_size)}
    for i, m in enumerate(["[0.00]", "[S01]", "[1.50]", "[S02]", "[3.25]", "[4.00]"]):
        del vocab[f"w{10 + i}"]
        vocab[m] = 10 + i
    del vocab[f"w{EOS}"]
    vocab["<|im_end|>"] = EOS
    tok = Tokenizer(models.WordLevel(vocab, unk_token="w0"))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    tok.add_special_tokens(["<|im_end|>"])
    return tok


def _host_embeds(gpu, prompts, audio, prec):
    H = gpu.cfg.hidden_size
    total = max(len(p) for p in prompts)
    rows = []
    for p, a in zip(prompts, audio):
        e = gpu.embed(np.asarray(p, dtype=np.uint32))
        if a is not None:
            t = torch.from_numpy(a)
            ar = (t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16) if prec == "bf16"
                  else t.to(torch.float16).numpy())
            k = 0
            for i, tok in enumerate(p):
                if tok == AUDIO:
                    e[i] = ar[k]
                    k += 1
        full = np.zeros((total, H), dtype=e.dtype)
        full[total - len(p):] = e
        rows.append(full)
    return np.stack(rows), [total - len(p) for p in prompts]


@pytest.mark.parametrize("prec", ["int8", "bf16"])
def test_transcribe_batch_matches_generate_and_parse(fmd, prec):
    print(f"[gpu] transcribe_batch facade {prec}", flush=True)
    cfg = tiny_cfg(fmd, layers=2, vocab=1024)
    gpu = fmd.Qwen3(cfg, prec, max_len=512).load(fmd.synthetic_weights(cfg, seed=71))
    tok = _tokenizer(cfg.vocab_size)
    rng = np.random.default_rng(72)
    reqs = []
    for i, n in enumerate([40, 25, 60, 33, 51]):
        ids = rng.integers(0, 1000, n)
        na = int(rng.integers(3, 9))
        at = rng.choice(np.arange(2, n - 2), na, replace=False)
        ids[at] = AUDIO
        audio = rng.standard_normal((na, cfg.hidden_size)).astype(np.float32)
        reqs.append(fmd.EncodedRequest(f"q{i}", ids.tolist(), audio, audio_seconds=float(n)))
    bad = fmd.EncodedRequest("bad", [AUDIO, 5, AUDIO], np.zeros((1, cfg.hidden_size), np.float32))
    reqs.insert(2, bad)
    force = [6, 9, 0, 4, 20, 7]
    budget = 24
    t = fmd.Transcriber(gpu, tok, AUDIO, fmd.EngineConfig(max_new_tokens=budget, max_batch_size=2,
                                                          eos_id=EOS))
    res, stats = t.transcribe_batch(reqs, raise_on_error=False, force_eot_step=force)
    assert isinstance(res[2], fmd.Failure) and "2 audio placeholders" in res[2].error
    assert stats.micro_batches == 3
    good = [i for i in range(len(reqs)) if i != 2]
    order = sorted(good, key=lambda i: len(reqs[i].prompt_ids))
    for g0 in range(0, len(order), 2):
        group = order[g0:g0 + 2]
        emb, pad = _host_embeds(gpu, [reqs[i].prompt_ids for i in group],
                                [reqs[i].audio for i in group], prec)
        want = gpu.generate_embeds(emb, pad, budget, eos=EOS, force_eot_step=[force[i] for i in group])
        for i, w in zip(group, want):
            r = res[i]
            assert isinstance(r, fmd.Response), (i, r)
            text = tok.decode(w.tokens, skip_special_tokens=True).strip()
            assert r.generated_tokens == len(w.tokens) and r.finish_reason == w.finish_reason
            assert r.text == text
            assert r.segments == fmd.transcript.parse(text)
            assert r.prompt_tokens == len(reqs[i].prompt_ids) and r.id == reqs[i].id
    # rows that would run past the RoPE table fail their whole micro-batch
    small = fmd.Qwen3(cfg, prec, max_len=64).load(fmd.synthetic_weights(cfg, seed=71))
    t2 = fmd.Transcriber(small, tok, AUDIO, fmd.EngineConfig(max_new_tokens=40, max_batch_size=4,
                                                             eos_id=EOS))
    res2, _ = t2.transcribe_batch(reqs[:2], raise_on_error=False)
    for r in res2:
        assert isinstance(r, fmd.Failure) and r.error.startswith("batch generation failed: rope")
    with pytest.raises(fmd.FmdError, match="batch generation failed"):
        t2.transcribe_batch(reqs[:2])


@pytest.mark.parametrize("prec", ["int8", "bf16"])
def test_transcribe_mel_encodes_then_transcribes(fmd, orc, prec):
    """transcribe_mel: every request's log-mel chunks through the device
    encoder + adaptor in one batched pass (engine.rs:329-346), then the same
    facade.  The responses equal transcribe_batch on requests carrying the
    encoder's own per-audio rows, and those rows match the oracle's
    encode_audio (mod.rs:82-126) at the audio dtype's bar."""
    print(f"[gpu] transcribe_mel {prec}", flush=True)
    cfg = tiny_cfg(fmd, layers=2, vocab=1024)
    gpu = fmd.Qwen3(cfg, prec, max_len=512).load(fmd.synthetic_weights(cfg, seed=73))
    acfg = fmd.AudioConfig(num_mel_bins=8, d_model=128, encoder_layers=2,
                           encoder_attention_heads=2, encoder_ffn_dim=256,
                           max_source_positions=24, adaptor_input_dim=512,
                           hidden_size=cfg.hidden_size, audio_merge_size=4, norm_eps=1e-6)
    aw = fmd.synthetic_audio_weights(acfg, seed=74)
    enc = fmd.AudioEncoder(acfg, prec).load(aw)
    tok = _tokenizer(cfg.vocab_size)
    rng = np.random.default_rng(75)
    reqs = []
    for i, chunks in enumerate([[6, 2], [4], [6, 6, 1], [3]]):
        mel = fmd.synthetic_mel(len(chunks), acfg, seed=80 + i)
        n_audio = sum(chunks)
        ids = rng.integers(0, 1000, 10 + n_audio + i)
        at = rng.choice(np.arange(1, len(ids) - 1), n_audio, replace=False)
        ids[at] = AUDIO
        reqs.append(fmd.MelRequest(f"m{i}", ids.tolist(), mel, chunks, audio_seconds=30.0 * len(chunks)))
    force = [5, 3, 9, 2]
    budget = 16
    t = fmd.Transcriber(gpu, tok, AUDIO, fmd.EngineConfig(max_new_tokens=budget, max_batch_size=3,
                                                          eos_id=EOS), encoder=enc, encoder_batch=2)
    res, stats = t.transcribe_mel(reqs, raise_on_error=False, force_eot_step=force)
    assert stats.encode_seconds > 0 and stats.micro_batches == 2
    mel_all = np.concatenate([np.asarray(r.mel) for r in reqs])
    tokens = [k for r in reqs for k in r.chunk_tokens]
    mapping = [i for i, r in enumerate(reqs) for _ in r.chunk_tokens]
    rows = enc.encode_audio(mel_all, tokens, mapping, len(reqs))
    enc_reqs = [fmd.EncodedRequest(r.id, r.prompt_ids, a, r.audio_seconds) for r, a in zip(reqs, rows)]
    want, _ = t.transcribe_batch(enc_reqs, raise_on_error=False, force_eot_step=force)
    for r, w in zip(res, want):
        assert isinstance(r, fmd.Response), r
        assert (r.text, r.generated_tokens, r.finish_reason) == (w.text, w.generated_tokens,
                                                                 w.finish_reason)
    ref = orc.OracleEncoder(acfg, {"int8": orc.F16, "bf16": orc.BF16}[prec]).load(aw)
    ref_rows = ref.encode_audio(mel_all, tokens, mapping, len(reqs))
    # f16: two rounding steps of the oracle's value, or 2e-2; bf16: four (the
    # adaptor's closing LayerNorm divides a one-step difference of its input
    # by the row's spread; test_gpu_encoder holds bf16 to the twin's floor)
    mant, steps = (7, 2) if prec == "bf16" else (10, 1)
    for r, a, b in zip(reqs, rows, ref_rows):
        got = (a.astype(np.uint32) << 16).view(np.float32) if prec == "bf16" else a.astype(np.float32)
        assert got.shape == b.shape == (sum(r.chunk_tokens), cfg.hidden_size)
        bar = np.maximum(2e-2, 2.0 ** (np.floor(np.log2(np.maximum(np.abs(b), 2.0 ** -14))) - mant + steps))
        assert np.all(np.abs(got - b) <= bar), float(np.max(np.abs(got - b)))
