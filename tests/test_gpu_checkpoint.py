"""A local checkpoint directory loads into the same decoder as the tensors
handed over directly: two bf16 shards plus tensors of the reference's other
modules (skipped), config.json's text_config, tied head.  Logits, the cache
and (int8) the Q8_0 blocks must be identical bit for bit."""
import dataclasses
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from tests.gpu_util import small_cfg

pytestmark = pytest.mark.gpu


def _checkpoint(fmd, tmp_path):
    cfg = small_cfg(fmd)
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
