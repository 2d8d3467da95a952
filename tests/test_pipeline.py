"""Host logic of the transcribe_batch facade (pipeline.py), with a stand-in
decoder that records the micro-batches it is given (no device needed):

- a request whose placeholders and audio rows disagree fails alone with
  splice_audio's message (mod.rs:145-150);
- the rest are sorted by prompt length, stably, and cut into micro-batches
  of max(max_batch_size, 1) (engine.rs:383-387);
- a micro-batch failure fails every member with "batch generation failed:
  {e}" (engine.rs:414-421);
- outputs are decoded without special tokens, trimmed and parsed
  (engine.rs:393-412, prompt.rs:153-155);
- raise_on_error raises on the first failed slot.
"""
import numpy as np
import pytest


def _tokenizer():
    from tokenizers import Tokenizer, models, pre_tokenizers

    words = ["[0.00]", "[S01]", "hello", "world", "[1.50]", "[S02]", "[2.25]", "again",
             "<|im_end|>"]
    vocab = {w: i for i, w in enumerate(words)}
    for i in range(len(words), 64):
        vocab[f"w{i}"] = i
    tok = Tokenizer(models.WordLevel(vocab, unk_token="w9"))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    tok.add_special_tokens(["<|im_end|>"])
    return tok


class _FakeModel:
    """Records micro-batches; emits the tokens of a table per prompt length."""

    def __init__(self, fmd, outputs, fail_lengths=()):
        self.fmd = fmd
        self.outputs = outputs
        self.fail_lengths = set(fail_lengths)
        self.batches = []

    def assemble(self, prompts, audio=None, audio_token_id=-1):
        self.batches.append([len(p) for p in prompts])
        total = max(len(p) for p in prompts)
        return np.zeros((len(prompts), total, 4)), [total - len(p) for p in prompts]

    def generate_device(self, embeds, pad, budget, eos, force_eot_step=None, chunk=256):
        lens = [embeds.shape[1] - p for p in pad]
        if self.fail_lengths & set(lens):
            raise self.fmd.FmdError(-1, "kv cache overflow: 0 + 9 exceeds capacity 8")
        return [self.fmd.Generated(list(self.outputs[n]), self.fmd.FinishReason.STOP) for n in lens]


AUDIO = 63


def _requests(fmd):
    r = []
    for i, n in enumerate([5, 3, 7, 3, 9, 4]):
        ids = [1] * n
        ids[0] = AUDIO
        r.append(fmd.EncodedRequest(f"r{i}", ids, np.zeros((1, 4), np.float32), audio_seconds=1.0 + i))
    r[2] = fmd.EncodedRequest("r2", [AUDIO, AUDIO, 1, 1, 1, 1, 1], np.zeros((1, 4), np.float32))
    return r


def test_facade_orders_chunks_decodes_and_parses(fmd):
    outputs = {5: [0, 1, 2, 3, 4, 8], 3: [5, 6], 9: [0, 5, 7, 6], 4: [8]}
    model = _FakeModel(fmd, outputs)
    t = fmd.Transcriber(model, _tokenizer(), AUDIO, fmd.EngineConfig(max_batch_size=2))
    res, stats = t.transcribe_batch(_requests(fmd), raise_on_error=False)
    # r2 has two placeholders and one audio row: it fails alone
    assert isinstance(res[2], fmd.Failure)
    assert res[2].error == "prompt has 2 audio placeholders but the encoder produced 1 embeddings"
    # stable sort by length: r1 (3), r3 (3), r5 (4), r0 (5), r4 (9) -> batches of 2
    assert model.batches == [[3, 3], [4, 5], [9]]
    assert stats.micro_batches == 3 and stats.requests == 6
    r0 = res[0]
    assert r0.text == "[0.00] [S01] hello world [1.50]"
    assert r0.segments == [fmd.transcript.Segment(0.0, 1.5, "S01", "hello world")]
    assert r0.generated_tokens == 6 and r0.prompt_tokens == 5 and r0.audio_seconds == 1.0
    assert res[1].text == "[S02] [2.25]" and res[1].segments == []
    assert res[5].text == "" and res[5].generated_tokens == 1
    assert stats.generated_tokens == 6 + 2 + 2 + 4 + 1


def test_facade_batch_failure_and_raise(fmd):
    outputs = {5: [2], 3: [3], 9: [2], 4: [3]}
    model = _FakeModel(fmd, outputs, fail_lengths=[9])
    t = fmd.Transcriber(model, _tokenizer(), AUDIO, fmd.EngineConfig(max_batch_size=2))
    res, _ = t.transcribe_batch(_requests(fmd), raise_on_error=False)
    assert res[4].error == "batch generation failed: kv cache overflow: 0 + 9 exceeds capacity 8"
    assert isinstance(res[0], fmd.Response) and res[0].text == "hello"
    # the binding raises RuntimeError("{id}: {e}") on the first failed slot
    # (fmd-py lib.rs:376-377)
    with pytest.raises(RuntimeError) as ei:
        t.transcribe_batch(_requests(fmd))
    assert isinstance(ei.value, fmd.FmdError)
    assert str(ei.value) == ("r2: prompt has 2 audio placeholders but the encoder produced 1 "
                             "embeddings")
