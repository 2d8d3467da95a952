"""Device-side prompt assembly against a numpy restatement of
MossTranscribeDiarize::splice_audio (mod.rs:128-180) and the engine's left
pad (engine.rs:476-491): text positions take their embedding row, audio
placeholders take the row's audio embeddings in order (rounded to the
activation dtype, round-to-nearest-even), pads are zero.  Bit-exact."""
import numpy as np
import pytest
import torch

from tests.gpu_util import tiny_cfg

pytestmark = pytest.mark.gpu

AUDIO = 1000


def _round(a32, prec):
    t = torch.from_numpy(np.ascontiguousarray(a32, dtype=np.float32))
    if prec == "bf16":
        return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return t.to(torch.float16).numpy()


def _restated(gpu, prompts, audio32, total, prec):
    H = gpu.cfg.hidden_size
    rows = []
    for p, a in zip(prompts, audio32):
        e = gpu.embed(np.asarray(p, dtype=np.uint32)) if len(p) else np.zeros((0, H), gpu.precision.numpy_storage)
        if a is not None:
            ar = _round(a, prec)
            k = 0
            for i, t in enumerate(p):
                if t == AUDIO:
                    e[i] = ar[k]
                    k += 1
        full = np.zeros((total, H), dtype=e.dtype)
        full[total - len(p):] = e
        rows.append(full)
    return np.stack(rows)


def _bits(x):
    return x.contiguous().view(torch.int16).cpu().numpy()


@pytest.fixture(scope="module")
def prompts():
    return [[5, AUDIO, AUDIO, 17, AUDIO, 9],            # audio runs split by a time marker
            [3, 4],
            [AUDIO, AUDIO, AUDIO, AUDIO, 7],
            []]


@pytest.mark.parametrize("prec", ["int8", "bf16"])
def test_assemble_matches_splice_and_pad(fmd, prompts, prec):
    print(f"[gpu] assemble {prec}", flush=True)
    cfg = tiny_cfg(fmd)
    gpu = fmd.Qwen3(cfg, prec, max_len=512).load(fmd.synthetic_weights(cfg, seed=2))
    rng = np.random.default_rng(4)
    audio32 = [rng.standard_normal((3, cfg.hidden_size)).astype(np.float32), None,
               rng.standard_normal((4, cfg.hidden_size)).astype(np.float32), None]
    want = _restated(gpu, prompts, audio32, 8, prec)
    # host f32 audio, a longer common length than the longest prompt
    out, pad = gpu.assemble(prompts, audio32, AUDIO, total=8)
    assert pad == [2, 6, 3, 8]
    assert np.array_equal(_bits(out), want.view(np.int16))
    # the same audio already in the activation dtype on the device
    dt = torch.bfloat16 if prec == "bf16" else torch.float16
    dev = [None if a is None else torch.from_numpy(a).to(dt).cuda() for a in audio32]
    out2, _ = gpu.assemble(prompts, dev, AUDIO, total=8)
    assert np.array_equal(_bits(out2), _bits(out))
    # prefill from the device block equals prefill from host embeddings
    live = prompts[:3]
    blk, pad = gpu.assemble(live, audio32[:3], AUDIO)
    host = _restated(gpu, live, audio32[:3], max(map(len, live)), prec)
    kv1 = gpu.new_caches(3, 16)
    kv2 = gpu.new_caches(3, 16)
    a = gpu.prefill_device(blk, kv1, pad)
    b = gpu.prefill(host, kv2, pad)
    assert np.array_equal(a, b)
    assert np.array_equal(kv1.read(0, 0), kv2.read(0, 0))


def test_assemble_rejects_what_the_reference_rejects(fmd, prompts):
    cfg = tiny_cfg(fmd)
    gpu = fmd.Qwen3(cfg, "bf16", max_len=512).load(fmd.synthetic_weights(cfg, seed=2))
    a = np.zeros((2, cfg.hidden_size), np.float32)
    with pytest.raises(fmd.FmdError, match="prompt has 3 audio placeholders but the encoder produced 2 embeddings"):
        gpu.assemble([prompts[0]], [a], AUDIO)
    with pytest.raises(fmd.FmdError, match="prompt has 1 audio placeholders but the encoder produced 0 embeddings"):
        gpu.assemble([[AUDIO, 3]], None, AUDIO)
    with pytest.raises(fmd.FmdError, match="token id out of range"):
        gpu.assemble([[cfg.vocab_size]], None, AUDIO)
    with pytest.raises(fmd.FmdError, match="longer than the assembled length"):
        gpu.assemble([[1, 2, 3]], None, AUDIO, total=2)
