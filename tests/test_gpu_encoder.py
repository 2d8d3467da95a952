"""The audio path on the device (fmd_enc_*: WhisperEncoder, VqAdaptor,
MossModel::encode_audio) against the oracle on the same seeded weights and
log-mel chunks.

Bars: f32 within 1e-4; f16 (the int8 precision's audio dtype) within 2e-2,
or one unit in the last place of the oracle's value where that is larger
(both round every op's output to the dtype; they differ only in f32
summation order, so a value may sit one rounding step apart).  bf16 at full
width: its 8-bit mantissa makes such one-step differences reach 2-3 steps
after a LayerNorm (which divides by the row's spread); there the device's
distance to the oracle must stay within 2x (max) and 1.5x (rms) of the
distance between the oracle and the torch twin (tests/torch_encoder_ref.py:
the same rounding points, BLAS summation), computed on the same input in the
same test, and the share of elements that differ within 2x the twin's.
Checked:

- the convolutional stem (mel cast, conv1 + gelu, conv2 + gelu, positions)
  and the final LayerNorm, at a tiny width and at Whisper-medium's (80 mels,
  3000 frames, d_model 1024) over two windows;
- two encoder layers at full width over two 1500-position windows, each layer
  fed the oracle's own input (no error carried from layer to layer), and the
  two together;
- one 30 s window through all 24 layers, f16;
- the adaptor on a full window's frames, and encode_audio's chunk trimming,
  per-audio joins and merge, bit-identical for every encoder batch size;
- the reference's argument errors.
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OP = {"f32": 0, "f16": 1, "bf16": 2}
PREC = {"f32": "f32", "f16": "int8", "bf16": "bf16"}   # library precision per audio dtype


def acfg(fmd, layers=2, **kw):
    base = dict(num_mel_bins=8, d_model=128, encoder_layers=layers, encoder_attention_heads=2,
                encoder_ffn_dim=256, max_source_positions=40, adaptor_input_dim=256,
                hidden_size=128, audio_merge_size=2, norm_eps=1e-6)
    base.update(kw)
    return fmd.AudioConfig(**base)


def full(fmd, layers):
    return fmd.AudioConfig(encoder_layers=layers)


def to_f32(a, dt):
    if dt == "bf16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def from_f32(x, dt, orc):
    return orc.to_storage(x, OP[dt])


def ulp(x, dt):
    if dt == "f32":
        return np.zeros_like(x)
    mant = 7 if dt == "bf16" else 10
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - mant)


def check(got, want, dt, what):
    d = np.abs(got - want)
    if dt == "f32":
        bar = np.maximum(1e-4, 1e-4 * np.abs(want))
    else:
        bar = np.maximum(2e-2, ulp(want, dt) * 1.0001)
    worst = float(np.max(d - bar))
    print(f"[gap] {what} {dt}: max |d| {float(d.max()):.4g}, rms {float(np.sqrt(np.mean(d * d))):.3g}, "
          f"max |x| {float(np.abs(want).max()):.3g}", flush=True)
    assert worst <= 0.0, (what, float(d.max()))


def check_floor(got, want, twin, what):
    """bf16: the device within the oracle-twin distance (see the module note)."""
    dg, dtw = np.abs(got - want), np.abs(twin - want)
    rg, rt = float(np.sqrt(np.mean(dg * dg))), float(np.sqrt(np.mean(dtw * dtw)))
    print(f"[gap] {what} bf16: device-oracle max {float(dg.max()):.4g} rms {rg:.3g} "
          f"(differing {float(np.mean(dg > 0)):.3%}); twin-oracle max {float(dtw.max()):.4g} "
          f"rms {rt:.3g} (differing {float(np.mean(dtw > 0)):.3%})", flush=True)
    assert float(dg.max()) <= max(2e-2, 2.0 * float(dtw.max())), what
    assert rg <= max(1e-4, 1.5 * rt), what
    assert float(np.mean(dg > 0)) <= 2.0 * float(np.mean(dtw > 0)) + 1e-3, what


def twin(cfg, w):
    import torch

    from tests.torch_encoder_ref import TorchWhisper

    return TorchWhisper(cfg, w, torch.bfloat16)


def pair(fmd, orc, cfg, dt, seed):
    w = fmd.synthetic_audio_weights(cfg, seed=seed)
    gpu = fmd.AudioEncoder(cfg, PREC[dt]).load(w)
    ref = orc.OracleEncoder(cfg, OP[dt]).load(w)
    return gpu, ref, w


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_stem_and_final_norm_tiny(fmd, orc, dt):
    print(f"[gpu] encoder stem tiny {dt}", flush=True)
    cfg = acfg(fmd, layers=0)
    gpu, ref, _ = pair(fmd, orc, cfg, dt, 1)
    mel = fmd.synthetic_mel(3, cfg, seed=2)
    check(to_f32(gpu.forward(mel), dt), ref.forward(mel), dt, "stem+norm tiny")
    # shorter chunks than the positions table (frames < 2 * max_source_positions)
    short = mel[:, :, :30]
    check(to_f32(gpu.forward(short), dt), ref.forward(short), dt, "stem+norm 30 frames")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_stem_full_width_two_windows(fmd, orc, dt):
    print(f"[gpu] encoder stem full width {dt}", flush=True)
    cfg = full(fmd, 0)
    gpu, ref, w = pair(fmd, orc, cfg, dt, 3)
    mel = fmd.synthetic_mel(2, cfg, seed=4)
    got = gpu.forward(mel)
    assert got.shape == (2, 1500, 1024)
    if dt == "bf16":
        import torch

        with torch.no_grad():
            tw = twin(cfg, w).forward(mel).numpy()
        check_floor(to_f32(got, dt), ref.forward(mel), tw, "stem+norm full")
    else:
        check(to_f32(got, dt), ref.forward(mel), dt, "stem+norm full")


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_layers_tiny(fmd, orc, dt):
    print(f"[gpu] encoder layers tiny {dt}", flush=True)
    cfg = acfg(fmd, layers=2)
    gpu, ref, _ = pair(fmd, orc, cfg, dt, 5)
    mel = fmd.synthetic_mel(3, cfg, seed=6)
    check(to_f32(gpu.forward(mel), dt), ref.forward(mel), dt, "encoder tiny")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_layers_full_width_two_windows(fmd, orc, dt):
    """Each of two layers fed the oracle's own input, then both together with
    the final norm, over two 1500-position windows at Whisper-medium width."""
    print(f"[gpu] encoder layers full width {dt}", flush=True)
    cfg = full(fmd, 2)
    gpu, ref, w = pair(fmd, orc, cfg, dt, 7)
    mel = fmd.synthetic_mel(2, cfg, seed=8)
    x0 = ref.stem(mel)
    x1 = ref.layers(x0, 0, 1)
    x2 = ref.layers(x1, 1, 1)
    if dt == "bf16":
        import torch

        tw = twin(cfg, w)
        for i, (xin, want) in enumerate(((x0, x1), (x1, x2))):
            got = to_f32(gpu.layers(from_f32(xin, dt, orc), i, 1), dt)
            with torch.no_grad():
                t_out = tw.layer(i, torch.from_numpy(xin)).numpy()
            check_floor(got, want, t_out, f"layer {i}")
        with torch.no_grad():
            t_all = tw.forward(mel, layers=2).numpy()
        check_floor(to_f32(gpu.forward(mel), dt), ref.forward(mel), t_all, "forward 2 layers")
        return
    for i, (xin, want) in enumerate(((x0, x1), (x1, x2))):
        got = to_f32(gpu.layers(from_f32(xin, dt, orc), i, 1), dt)
        check(got, want, dt, f"layer {i}")
    got = to_f32(gpu.layers(from_f32(x0, dt, orc), 0, 2, final_norm=True), dt)
    check(got, ref.layers(x0, 0, 2, final_norm=True), dt, "layers 0-1 + norm")
    check(to_f32(gpu.forward(mel), dt), ref.forward(mel), dt, "forward 2 layers")


def test_full_depth_window_f16(fmd, orc):
    """One 30 s window through the stem, all 24 layers and the final norm
    (Whisper-medium shape, the int8 precision's f16 audio path)."""
    print("[gpu] encoder full depth f16", flush=True)
    cfg = full(fmd, 24)
    gpu, ref, _ = pair(fmd, orc, cfg, "f16", 9)
    mel = fmd.synthetic_mel(1, cfg, seed=10)
    check(to_f32(gpu.forward(mel), "f16"), ref.forward(mel), "f16", "24 layers")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_adaptor_full_window(fmd, orc, dt):
    print(f"[gpu] adaptor full window {dt}", flush=True)
    cfg = full(fmd, 0)
    gpu, ref, w = pair(fmd, orc, cfg, dt, 11)
    frames = orc.round_to(np.random.default_rng(12).standard_normal((1500, 1024)).astype(np.float32),
                          OP[dt])
    got = gpu.merge_and_project(from_f32(frames, dt, orc))
    assert got.shape == (375, 1024)
    if dt == "bf16":
        import torch

        with torch.no_grad():
            tw = twin(cfg, w).adaptor(frames).numpy()
        check_floor(to_f32(got, dt), ref.adaptor(frames), tw, "adaptor")
    else:
        check(to_f32(got, dt), ref.adaptor(frames), dt, "adaptor")
    # a trailing partial group is dropped (adaptor.rs:41-52)
    assert gpu.merge_and_project(from_f32(frames[:7], dt, orc)).shape == (1, 1024)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_encode_audio_reassembly(fmd, orc, dt):
    """mod.rs:82-126 over five chunks of three audios: each chunk trimmed to
    its tokens * merge frames (all of them when it asks for more), joined per
    audio in chunk order, merged and projected; the same bits for encoder
    batches of 1, 2 and 16 chunks."""
    print(f"[gpu] encode_audio {dt}", flush=True)
    cfg = acfg(fmd, layers=1)
    gpu, ref, _ = pair(fmd, orc, cfg, dt, 13)
    mel = fmd.synthetic_mel(5, cfg, seed=14)
    tokens = [20, 7, 3, 30, 11]     # 40 frames per chunk, merge 2: 30 tokens keep all 40
    mapping = [0, 1, 0, 2, 1]
    outs = [gpu.encode_audio(mel, tokens, mapping, 3, encoder_batch=b) for b in (1, 2, 16)]
    for o in outs[1:]:
        for a in range(3):
            assert np.array_equal(o[a], outs[0][a])
    want = ref.encode_audio(mel, tokens, mapping, 3)
    assert [o.shape[0] for o in outs[0]] == [20 + 3, 7 + 11, 20]
    for a in range(3):
        check(to_f32(outs[0][a], dt), want[a], dt, f"audio {a}")
    offs = gpu.encode_offsets(tokens, mapping, 3, 80)
    assert offs.tolist() == [0, 23, 41, 61]


def test_encoder_argument_errors(fmd):
    cfg = acfg(fmd, layers=1)
    gpu = fmd.AudioEncoder(cfg, "bf16").load(fmd.synthetic_audio_weights(cfg, seed=15))
    mel = fmd.synthetic_mel(2, cfg, seed=16)
    with pytest.raises(fmd.FmdError, match="chunk_mapping"):
        gpu.encode_audio(mel, [1, 1], [0, 3], 2)
    with pytest.raises(fmd.FmdError, match="even"):
        gpu.forward(mel[:, :, :21])
    with pytest.raises(fmd.FmdError, match="exceeds"):
        gpu.forward(np.zeros((1, cfg.num_mel_bins, 2 * cfg.max_source_positions + 2), np.float32))
    with pytest.raises(fmd.FmdError, match="head_dim"):
        fmd.AudioEncoder(acfg(fmd, encoder_attention_heads=4), "bf16")
    incomplete = fmd.AudioEncoder(cfg, "bf16")
    with pytest.raises(fmd.FmdError, match="incomplete"):
        incomplete.forward(mel)
    with pytest.raises(fmd.FmdError, match="unknown tensor"):
        incomplete.set_weight("model.whisper_encoder.layers.0.self_attn.k_proj.bias",
                              np.zeros(cfg.d_model, np.float32))
    assert math.isclose(cfg.head_dim(), 64)


def test_windows_are_independent_of_the_batch(fmd, orc):
    """Twelve windows at Whisper-medium width in one pass (18,012 rows, all
    in 256-row tiles) against each window alone (1,501 rows: 128- and 64-row
    tiles): the same bits, since every tile kind sums each output over k in
    the same order, applies the same epilogue steps (the residual ones
    included), and nothing crosses a window."""
    print("[gpu] encoder batch independence (tile kinds)", flush=True)
    cfg = full(fmd, 2)
    w = fmd.synthetic_audio_weights(cfg, seed=17)
    gpu = fmd.AudioEncoder(cfg, "bf16").load(w)
    mel = fmd.synthetic_mel(12, cfg, seed=18)
    together = gpu.forward(mel)
    for i in (0, 5, 11):
        alone = gpu.forward(mel[i:i + 1])
        assert np.array_equal(together[i], alone[0]), i
