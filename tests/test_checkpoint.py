"""Local checkpoint ingest on the CPU: directory resolution (hub.rs:88-133),
text_config defaults (config.rs:8-41), which tensors reach the decoder and in
which dtype (qwen3.rs:354-390, 566-578; linear.rs:102-153).  The decoder is
replaced by a recorder, so no device is needed."""
import json

import pytest
import torch
from safetensors.torch import save_file

TEXT = {"vocab_size": 64, "hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 1,
        "num_attention_heads": 4, "num_key_value_heads": 2}


class Recorder:
    def __init__(self):
        self.seen = []

    def set_weight(self, name, t):
        self.seen.append((name, t.dtype, tuple(t.shape), t.clone()))


def _write_config(d, **extra):
    (d / "config.json").write_text(json.dumps({"text_config": dict(TEXT, **extra), "audio_token_id": 7}))


def test_resolve_local_errors(fmd, tmp_path):
    ck = fmd.checkpoint
    with pytest.raises(fmd.CheckpointError, match="not a directory"):
        ck.resolve_local(tmp_path / "absent")
    with pytest.raises(fmd.CheckpointError, match="no .safetensors weights found"):
        ck.resolve_local(tmp_path)
    save_file({"x": torch.zeros(2)}, str(tmp_path / "b.safetensors"))
    save_file({"y": torch.zeros(2)}, str(tmp_path / "a.safetensors"))
    with pytest.raises(fmd.CheckpointError, match="config.json is missing"):
        ck.resolve_local(tmp_path)
    _write_config(tmp_path)
    cfg, files = ck.resolve_local(tmp_path)
    assert cfg.name == "config.json"
    assert [f.name for f in files] == ["a.safetensors", "b.safetensors"]   # sorted by path


def test_text_config_defaults_and_overrides(fmd, tmp_path):
    ck = fmd.checkpoint
    c = ck.text_config({"text_config": TEXT})
    assert (c.head_dim, c.rms_norm_eps, c.rope_theta, c.max_position_embeddings) == (128, 1e-6, 1e6, 131072)
    assert not c.tie_word_embeddings and not c.attention_bias
    c = ck.text_config({"text_config": dict(TEXT, head_dim=64, rope_theta=5e5, tie_word_embeddings=True)})
    assert (c.head_dim, c.rope_theta, c.tie_word_embeddings) == (64, 5e5, True)
    with pytest.raises(fmd.CheckpointError, match="no text_config"):
        ck.text_config({"audio_config": {}})
    bad = dict(TEXT)
    del bad["num_key_value_heads"]
    with pytest.raises(fmd.CheckpointError, match="num_key_value_heads"):
        ck.text_config({"text_config": bad})


def test_only_decoder_tensors_in_stored_dtype(fmd, tmp_path):
    ck = fmd.checkpoint
    P = "model.language_model."
    g = torch.Generator().manual_seed(0)
    a = {P + "embed_tokens.weight": torch.randn(64, 256, generator=g).to(torch.bfloat16),
         P + "norm.weight": torch.ones(256, dtype=torch.float32),
         "model.whisper_encoder.conv1.weight": torch.zeros(4, 4),
         "lm_head.weight": torch.randn(64, 256, generator=g).to(torch.bfloat16)}
    b = {P + "layers.0.mlp.down_proj.weight": torch.randn(256, 512, generator=g).to(torch.float16),
         P + "layers.0.self_attn.q_norm.weight": torch.ones(128, dtype=torch.float64),
         "model.vq_adaptor.fc.weight": torch.zeros(2, 2)}
    save_file(a, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(b, str(tmp_path / "model-00002-of-00002.safetensors"))
    _write_config(tmp_path)
    _, files = ck.resolve_local(tmp_path)
    r = Recorder()
    assert ck.load_into(r, files) == 5
    got = {n: (dt, shp, t) for n, dt, shp, t in r.seen}
    assert set(got) == {P + "embed_tokens.weight", P + "norm.weight", "lm_head.weight",
                        P + "layers.0.mlp.down_proj.weight", P + "layers.0.self_attn.q_norm.weight"}
    # stored 16-bit and f32 tensors pass through unchanged; f64 is widened to f32
    assert got[P + "embed_tokens.weight"][0] == torch.bfloat16
    assert torch.equal(got[P + "embed_tokens.weight"][2], a[P + "embed_tokens.weight"])
    assert got[P + "layers.0.mlp.down_proj.weight"][0] == torch.float16
    assert got[P + "layers.0.self_attn.q_norm.weight"][0] == torch.float32
    assert got["lm_head.weight"][0] == torch.bfloat16


def test_prefixed_head_wins_and_duplicates_fail(fmd, tmp_path):
    ck = fmd.checkpoint
    P = "model.language_model."
    save_file({"lm_head.weight": torch.zeros(64, 256),
               P + "lm_head.weight": torch.ones(64, 256)}, str(tmp_path / "m.safetensors"))
    _write_config(tmp_path)
    _, files = ck.resolve_local(tmp_path)
    r = Recorder()
    assert ck.load_into(r, files) == 1
    assert r.seen[0][0] == P + "lm_head.weight"      # qwen3.rs:360-365 looks under the prefix first
    save_file({P + "norm.weight": torch.ones(256)}, str(tmp_path / "n1.safetensors"))
    save_file({P + "norm.weight": torch.ones(256)}, str(tmp_path / "n2.safetensors"))
    _, files = ck.resolve_local(tmp_path)
    with pytest.raises(fmd.CheckpointError, match="appears in"):
        ck.load_into(Recorder(), files)


def test_generation_config_defaults_and_budget(fmd, tmp_path):
    """generation_config.json (config.rs:91-117): absent -> the reference's
    Default (eos 151645, cap 5120); present -> its eos_token_id (else 151645,
    engine.rs:246) and max_new_tokens (else 5120); the engine's budget is
    min(max_new_tokens, max(cap, 1)) (engine.rs:466-469)."""
    import json

    g = fmd.generation_config(tmp_path)
    assert (g.bos_token_id, g.eos_token_id, g.pad_token_id, g.max_new_tokens) == (
        151643, 151645, 151643, 5120)
    cfg = fmd.engine_config(tmp_path)
    assert cfg.eos_id == 151645 and cfg.budget() == 4096
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": 7,
                                                                "max_new_tokens": 20}))
    cfg = fmd.engine_config(tmp_path, max_new_tokens=64, max_batch_size=3)
    assert cfg.eos_id == 7 and cfg.budget() == 20 and cfg.max_batch_size == 3
    assert fmd.engine_config(tmp_path, max_new_tokens=10).budget() == 10
    (tmp_path / "generation_config.json").write_text(json.dumps({"bos_token_id": 1}))
    g = fmd.generation_config(tmp_path)
    assert g.eos_token_id is None and g.pad_token_id is None and g.max_new_tokens == 5120
    assert fmd.engine_config(tmp_path).eos_id == 151645
    (tmp_path / "generation_config.json").write_text(json.dumps({"max_new_tokens": 0}))
    assert fmd.engine_config(tmp_path).budget() == 1   # max(0, 1)
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": -3}))
    with pytest.raises(fmd.CheckpointError, match="eos_token_id"):
        fmd.generation_config(tmp_path)
