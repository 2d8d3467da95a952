"""A local checkpoint directory loads into the same decoder as the tensors
handed over directly: two bf16 shards plus tensors of the reference's other
modules (skipped), config.json's text_config, tied head.  Logits, the cache
and (int8) the Q8_0 blocks must be identical bit for bit.  And the
checkpoint-loaded decoder agrees with the oracle loaded from the same shards
(read with safetensors' loader, the stored bf16 widened to f32 as the
reference's f32 source view does, linear.rs:126-134): prefill and decode
logits within 2e-2, greedy ids equal wherever the top-2 margin exceeds it
(int8 on two layers, bf16 on one)."""
import dataclasses
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from tests.gpu_util import OPREC, TOL, small_cfg

pytestmark = pytest.mark.gpu


def _checkpoint(fmd, tmp_path, layers=2):
    cfg = small_cfg(fmd, layers=layers)
    w = fmd.synthetic_weights(cfg, seed=11)
    bf = {n: torch.from_numpy(a).to(torch.bfloat16) for n, a in w.items()}
    names = sorted(bf)
    half = len(names) // 2
    save_file({n: bf[n] for n in names[:half]}, str(tmp_path / "model-00001-of-00002.safetensors"))
    rest = {n: bf[n] for n in names[half:]}
    rest["model.whisper_encoder.conv1.weight"] = torch.zeros(8, 4)
    save_file(rest, str(tmp_path / "model-00002-of-00002.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps(
        {"text_config": dataclasses.asdict(cfg), "audio_token_id": 151654}))
    return cfg, bf


@pytest.mark.parametrize("prec", ["int8", "bf16"])
def test_checkpoint_directory_matches_direct_load(fmd, tmp_path, prec):
    print(f"[gpu] checkpoint ingest {prec}", flush=True)
    cfg, bf = _checkpoint(fmd, tmp_path)
    a = fmd.load_checkpoint(tmp_path, prec, max_len=2048)
    b = fmd.Qwen3(cfg, prec, max_len=2048).load(bf)
    assert a.cfg == b.cfg
    assert a.weight_bytes() == b.weight_bytes()
    if prec == "int8":
        for name in ["model.language_model.layers.0.self_attn.q_proj.weight",
                     "model.language_model.layers.1.mlp.down_proj.weight",
                     "model.language_model.lm_head.weight"]:
            assert np.array_equal(a.q8_0_blocks(name), b.q8_0_blocks(name)), name
    rng = np.random.default_rng(3)
    lens = [300, 77, 512, 1]
    T = max(lens)
    ids = rng.integers(0, cfg.vocab_size, (4, T))
    outs = []
    for m in (a, b):
        e = m.embed(ids.reshape(-1)).reshape(4, T, -1)
        for r in range(4):
            e[r, :T - lens[r]] = 0
        kv = m.new_caches(4, T + 8)
        lg = m.prefill(e, kv, [T - n for n in lens], chunk=256)
        nxt = m.decode_step(lg.argmax(-1).tolist(), kv, [T - n for n in lens])
        outs.append((lg, nxt, kv.read(1, 0), kv.read(1, 1)))
    for x, y in zip(outs[0], outs[1]):
        assert np.array_equal(x, y)


def _oracle_from_directory(fmd, orc, directory, prec, max_len):
    """The oracle loaded from a checkpoint directory's decoder tensors."""
    from safetensors import safe_open

    config, shards = fmd.checkpoint.resolve_local(directory)
    cfg = fmd.checkpoint.text_config(config)
    ref = orc.OracleModel(cfg, OPREC[prec], max_len)
    tensors = {}
    for f in shards:
        with safe_open(str(f), framework="pt", device="cpu") as fh:
            for n in fh.keys():
                if fmd.checkpoint.decoder_tensor(n):
                    tensors[n] = fh.get_tensor(n).float().numpy()
    return ref.load(tensors), cfg


# bf16 on one layer: over two bf16 layers, summation-order differences
# between any two implementations already reach ~0.02 in the logits (the
# layer-by-layer decode test holds every layer to the bar on its own); the
# loading itself -- names, dtype views, tied head -- does not depend on depth,
# and the two-layer bf16 load is compared bit for bit with a direct load above.
@pytest.mark.parametrize("prec,layers", [("int8", 2), ("bf16", 1)])
def test_checkpoint_directory_matches_oracle(fmd, orc, tmp_path, prec, layers):
    print(f"[gpu] checkpoint ingest vs oracle {prec}, {layers} layers", flush=True)
    _checkpoint(fmd, tmp_path, layers=layers)
    gpu = fmd.load_checkpoint(tmp_path, prec, max_len=2048)
    ref, cfg = _oracle_from_directory(fmd, orc, tmp_path, prec, 2048)
    assert cfg == gpu.cfg
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in (300, 77, 512, 1)]
    emb, pad = ref.padded_embeds(prompts)
    gkv = gpu.new_caches(4, emb.shape[1] + 8)
    rkv = ref.new_kv(4, emb.shape[1] + 8)
    g = gpu.prefill(orc.to_storage(emb, OPREC[prec]), gkv, pad, chunk=256)
    r = ref.prefill(rkv, emb, pad, block=256)
    ids = r.argmax(-1).tolist()
    g2 = gpu.decode_step(ids, gkv, pad)
    r2 = ref.decode_step(rkv, ids, pad)
    for got, want in ((g, r), (g2, r2)):
        d = float(np.max(np.abs(got - want)))
        print(f"[gap] checkpoint {prec}: max |dlogit| {d:.4g}", flush=True)
        assert d < TOL[prec], d
        s = np.sort(want, axis=-1)
        for b in range(4):
            if s[b, -1] - s[b, -2] > TOL[prec]:
                assert int(got[b].argmax()) == int(want[b].argmax()), b


def test_generation_config_sets_eos_and_cap(fmd, tmp_path):
    """A checkpoint whose generation_config.json names an end-of-turn id and a
    cap of 20 tokens: the engine built from the directory stops a row at that
    id without emitting it (engine.rs:246, 508-520) and gives no row more
    than 20 tokens even when asked for 64 (engine.rs:466-469)."""
    print("[gpu] generation_config.json eos + cap", flush=True)
    _checkpoint(fmd, tmp_path, layers=2)
    gpu = fmd.load_checkpoint(tmp_path, "int8", max_len=4096)
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, gpu.cfg.vocab_size, n).tolist() for n in (90, 33, 140)]
    # a reference run whose end-of-turn id none of the rows emits in 64 steps
    for unused in range(gpu.cfg.vocab_size - 1, gpu.cfg.vocab_size - 9, -1):
        free = fmd.Engine(gpu, fmd.EngineConfig(max_new_tokens=64, max_batch_size=3,
                                                eos_id=unused))
        base, _ = free.generate(prompts)
        if all(len(b.tokens) == 64 for b in base):
            break
    assert all(len(b.tokens) == 64 for b in base)
    # an id that some row emits for the first time at a step in [1, 20) (the
    # first token of row 0 if none)
    row, step = next(((r, i) for r in range(3) for i in range(1, 20)
                      if base[r].tokens[i] not in base[r].tokens[:i]), (0, 0))
    eos = int(base[row].tokens[step])
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": eos,
                                                                "max_new_tokens": 20}))
    cfg = fmd.engine_config(tmp_path, max_new_tokens=64, max_batch_size=3)
    assert cfg.eos_id == eos and cfg.budget() == 20
    res, stats = fmd.Engine(gpu, cfg).generate(prompts)
    assert res[row].tokens == base[row].tokens[:step]
    assert res[row].finish_reason == fmd.FinishReason.STOP
    for r, b in zip(res, base):
        cut = b.tokens.index(eos) if eos in b.tokens[:20] else None
        if cut is None:
            assert r.tokens == b.tokens[:20] and r.finish_reason == fmd.FinishReason.LENGTH
        else:
            assert r.tokens == b.tokens[:cut] and r.finish_reason == fmd.FinishReason.STOP
    assert all(len(r.tokens) <= 20 for r in res)
