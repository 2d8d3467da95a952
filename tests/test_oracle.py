"""Pins the CPU oracle (the checker) before anything is compared against it.

Sources of truth, in order: the reference's own unit-test known answers
(qwen3.rs:601-820, linear.rs:337-364, engine.rs:601-615, config.rs:244-264),
values fixed by construction or closed form (Q8_0 blocks with exact scales,
round-half-away ties, RMSNorm of [3, 4], RoPE at position 0), library
routines (numpy / torch IEEE conversions), and a second, independent decoder
restatement in torch (tests/torch_ref.py).
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


# --------------------------------------------------------------------------
# IEEE conversions vs numpy / torch
# --------------------------------------------------------------------------

def _special_f32():
    bits = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x477FE000, 0x477FF000,
            0x477FEFFF, 0x47800000, 0x387FC000, 0x33800000, 0x33000000, 0x33000001,
            0x3F800000, 0x3F801000, 0x3F803000, 0x00000001, 0x007FFFFF, 0x38800000]
    return np.array(bits, dtype=np.uint32).view(np.float32)


def test_f16_conversion_matches_numpy(orc):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), _special_f32(),
                        rng.standard_normal(100_000).astype(np.float32) * 1e-5])
    x = x[~np.isnan(x)]
    got = orc.round_to(x, orc.F16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bf16_conversion_matches_torch(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), _special_f32()])
    x = x[~np.isnan(x)]
    got = orc.round_to(x, orc.BF16)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------------------
# Q8_0 (QTensor::quantize via linear.rs:194-201, 239-251)
# --------------------------------------------------------------------------

def _blk(d_bits, qs):
    return bytes([d_bits & 0xFF, d_bits >> 8]) + bytes(np.asarray(qs, dtype=np.int8).view(np.uint8))


def test_q8_0_known_answers(orc):
    """Blocks whose answer is fixed by construction; the cases are in
    tests/golden/q8_0_known_answers.json together with how each was derived."""
    cases = json.loads((GOLDEN / "q8_0_known_answers.json").read_text())["cases"]
    assert len(cases) >= 8
    for c in cases:
        x = np.array(c["x"], dtype=np.float32)[None, :]
        got = orc.quantize_q8_0(x)[0, 0].tobytes()
        want = _blk(int(c["d_bits"], 16), c["q"])
        assert got == want, c["name"]


def test_q8_0_ties_round_half_away_from_zero(orc):
    # d = 1 exactly (amax 127): x * id == x, so q = round(x) with Rust's f32::round.
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
    q = orc.quantize_q8_0(x[None])[0, 0, 2:].view(np.int8)
    assert list(q[:9]) == [127, 1, -1, 2, -2, 3, -3, 127, -127]  # half-to-even would give 0,0,2,-2,2,-2,126,-126


def test_q8_0_subnormal_and_overflowing_scales(orc):
    # amax = 127 * 2^-20 -> d = 2^-20, an f16 subnormal: 2^-20 / 2^-24 = 16 -> 0x0010
    x = (np.arange(-16, 16, dtype=np.float32) * np.float32(2.0**-20))
    x[0] = np.float32(127 * 2.0**-20)
    blk = orc.quantize_q8_0(x[None])[0, 0]
    assert int(blk[0]) | (int(blk[1]) << 8) == 0x0010
    assert list(blk[2:].view(np.int8)) == [127] + list(range(-15, 16))
    # amax = 127 * 2^17 -> d = 131072 > 65504: f16 overflows to +inf (0x7c00)
    y = np.zeros(32, dtype=np.float32)
    y[3] = np.float32(127 * 2.0**17)
    y[4] = -np.float32(2.0**17)
    blk = orc.quantize_q8_0(y[None])[0, 0]
    assert int(blk[0]) | (int(blk[1]) << 8) == 0x7C00
    assert blk[2:].view(np.int8)[3] == 127 and blk[2:].view(np.int8)[4] == -1


def test_q8_0_concat_equals_rowwise(orc):
    """cat(quantize) == quantize(cat) along the out axis (linear.rs:217-219)."""
    rng = np.random.default_rng(2)
    a = rng.standard_normal((7, 96)).astype(np.float32) * 0.02
    b = rng.standard_normal((5, 96)).astype(np.float32) * 0.02
    joined = orc.quantize_q8_0(np.concatenate([a, b]))
    parts = np.concatenate([orc.quantize_q8_0(a), orc.quantize_q8_0(b)])
    assert np.array_equal(joined, parts)


def test_q8_0_matches_numpy_restatement_of_ggml(orc):
    """GGML quantize_row_q8_0_ref restated with numpy float32 scalars and an
    exact (float64) half-away rounding, on random rows."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 256)) * rng.uniform(1e-4, 10, (64, 1))).astype(np.float32)
    blocks = orc.quantize_q8_0(x)
    xb = x.reshape(64, 8, 32)
    amax = np.abs(xb).max(axis=-1)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = (xb * inv[..., None]).astype(np.float32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    dbits = d.astype(np.float16).view(np.uint16)
    assert np.array_equal(blocks[..., 0] | (blocks[..., 1].astype(np.uint16) << 8), dbits)
    assert np.array_equal(blocks[..., 2:].view(np.int8), q)


def test_q8_0_dequantisation_is_exact(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    blocks = orc.quantize_q8_0(x)
    deq = orc.dequantize_q8_0(blocks, 4, 64)
    d = blocks[..., 0:2].copy().view(np.float16).astype(np.float32)  # (4, 2, 1)
    want = (d * blocks[..., 2:].view(np.int8).astype(np.float32)).reshape(4, 64)
    assert np.array_equal(deq, want)
    assert np.max(np.abs(deq - x)) <= np.max(np.abs(x)) / 127 * 0.5 * 1.01


# --------------------------------------------------------------------------
# Mask, RoPE, attention regrouping (qwen3.rs tests)
# --------------------------------------------------------------------------

def test_no_query_row_is_fully_masked(orc):
    """qwen3.rs:722-748."""
    m = orc.build_mask(2, 2, 0, 6, 6, [4, 0])[:, 0]
    assert np.isfinite(m).any(axis=-1).all()
    assert np.isinf(m[0, 4, :4]).all() and m[0, 4, 4] == 0 and np.isinf(m[0, 4, 5])


def test_softmax_over_the_mask_never_produces_nan(orc):
    """qwen3.rs:750-761."""
    m = torch.from_numpy(orc.build_mask(2, 2, 0, 6, 6, [4, 0]))
    assert torch.isfinite(torch.softmax(torch.zeros(2, 1, 12, 6) + m, dim=-1).sum())


def test_mask_is_tiled_for_the_regrouped_queries(orc):
    """qwen3.rs:763-777: rows repeat*q_len, row r*q_len+q carries query q."""
    m = orc.build_mask(1, 2, 0, 3, 3, [0])
    assert m.shape == (1, 1, 6, 3)
    for q in range(3):
        assert np.array_equal(m[0, 0, q], m[0, 0, 3 + q])


def test_mask_blocks_future_and_padding(orc):
    """qwen3.rs:799-820."""
    m = orc.build_mask(2, 2, 0, 4, 4, [2, 0])[:, 0]
    assert np.isinf(m[0, 2, 0]) and np.isinf(m[0, 2, 1]) and m[0, 2, 2] == 0 and np.isinf(m[0, 2, 3])
    assert list(m[1, 2, :3]) == [0, 0, 0] and np.isinf(m[1, 2, 3])


def test_rope_tables_closed_form(orc):
    c, s = orc.rope_tables(128, 1e6, 64, orc.F32)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # inv_freq[0] = 1: column 0 is cos(p), sin(p) in f32
    p = np.arange(64, dtype=np.float32)
    assert np.allclose(c[:, 0], np.cos(p), atol=1e-7) and np.allclose(s[:, 0], np.sin(p), atol=1e-7)
    # inv_freq[i] = theta^(-2i/hd) -> the last column at p = 50
    f = np.float32(50) * np.float32(1.0 / 1e6 ** (126 / 128))
    assert abs(c[50, 63] - math.cos(f)) < 1e-7


def test_rope_is_shift_invariant(orc):
    """qwen3.rs:650-673: the score depends only on the relative distance."""
    c, s = orc.rope_tables(4, 10_000.0, 32, orc.F32)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 1, 1, 4)).astype(np.float32)
    k = rng.standard_normal((1, 1, 1, 4)).astype(np.float32)

    def score(qp, kp):
        return float((orc.rope_apply(q, qp, c, s) * orc.rope_apply(k, kp, c, s)).sum())

    assert abs(score(5, 2) - score(20, 17)) < 1e-4
    assert abs(score(5, 2) - score(5, 3)) > 1e-3  # and it does depend on the distance


def test_rope_rotates_halves_not_interleaved_pairs(orc):
    """Rope::apply uses candle's rotate-half `rope` (qwen3.rs:139-144), pairing
    dims (i, i + hd/2).  A unit vector at dim i < 64 comes out as cos at i and
    sin at i + 64; at dim i + 64 as -sin at i and cos at i + 64; every other
    element stays 0.  An interleaved (rope_i) convention, which pairs (2i,
    2i + 1) and is shift-invariant too, fails this."""
    hd, theta, pos = 128, 1e6, 37
    c, s = orc.rope_tables(hd, theta, pos + 1, orc.F32)
    for i in (0, 1, 17, 63):
        x = np.zeros((1, 1, 1, hd), dtype=np.float32)
        x[..., i] = 1.0
        y = orc.rope_apply(x, pos, c, s).reshape(-1)
        want = np.zeros(hd, dtype=np.float32)
        want[i], want[i + 64] = c[pos, i], s[pos, i]
        assert np.array_equal(y, want), i
        x[..., i], x[..., i + 64] = 0.0, 1.0
        y = orc.rope_apply(x, pos, c, s).reshape(-1)
        want[:] = 0.0
        want[i], want[i + 64] = -s[pos, i], c[pos, i]
        assert np.array_equal(y, want), i
    # and the table entries are cos / sin of pos * theta^(-2i/hd) (f32 product)
    for i in (0, 17, 63):
        f = np.float32(pos) * np.float32(1.0 / theta ** (2 * i / hd))
        assert abs(c[pos, i] - math.cos(f)) < 1e-6 and abs(s[pos, i] - math.sin(f)) < 1e-6


def test_layer_by_layer_decode_composes_to_decode_step(fmd, orc):
    """decode_step (qwen3.rs:499-511) is embed, every Layer::forward at the
    same offset, the final norm and the logits: or_layer_decode over the
    layers then or_final_logits gives its logits and cache bit for bit."""
    cfg = fmd.TextConfig(vocab_size=512, hidden_size=256, intermediate_size=512,
                         num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2,
                         head_dim=128, rope_theta=1e6)
    w = fmd.synthetic_weights(cfg, seed=3)
    for prec in (orc.F32, orc.BF16, orc.INT8):
        ref = orc.OracleModel(cfg, prec, 128).load(w)
        pad = [3, 0, 7]
        a, b = ref.new_kv(3, 64), ref.new_kv(3, 64)
        a.fill_random(4, 20)
        b.fill_random(4, 20)
        ids = [5, 77, 300]
        want = ref.decode_step(a, ids, pad)
        x = orc.round_to(ref.embed(ids), prec)
        for layer in range(cfg.num_hidden_layers):
            x = ref.layer_decode(b, layer, x, pad)
        got = ref.final_logits(x)
        assert np.array_equal(got, want), prec
        for layer in range(cfg.num_hidden_layers):
            for which in (0, 1):
                assert np.array_equal(a.read(layer, which), b.read(layer, which))


def test_grouped_attention_matches_expanded_attention(orc):
    """qwen3.rs:682-714: regrouped queries == repeat_kv-expanded heads (1e-5)."""
    rng = np.random.default_rng(6)
    b, kvh, rep, t, L, d = 2, 3, 2, 4, 7, 5
    q = rng.standard_normal((b, kvh * rep, t, d)).astype(np.float32)
    k = rng.standard_normal((b, kvh, L, d)).astype(np.float32)
    v = rng.standard_normal((b, kvh, L, d)).astype(np.float32)
    got = orc.attention(q, k, v, None, L)
    kk = torch.from_numpy(k).repeat_interleave(rep, dim=1)
    vv = torch.from_numpy(v).repeat_interleave(rep, dim=1)
    sc = (torch.from_numpy(q) @ kk.transpose(-1, -2)) * (1.0 / math.sqrt(d))
    want = (torch.softmax(sc, -1) @ vv).transpose(1, 2).reshape(b, t, -1).numpy()
    assert np.max(np.abs(got - want)) < 1e-5


def test_repeat_kv_ordering(orc):
    """qwen3.rs:635-648: query head h reads kv head h // repeat (not interleaved)."""
    b, kvh, rep, L, d = 1, 2, 2, 1, 2
    k = np.zeros((b, kvh, L, d), dtype=np.float32)
    v = np.array([1, 2, 3, 4], dtype=np.float32).reshape(b, kvh, L, d)
    q = np.zeros((b, kvh * rep, 1, d), dtype=np.float32)
    out = orc.attention(q, k, v, None, L).reshape(-1)
    assert list(out) == [1, 2, 1, 2, 3, 4, 3, 4]


# --------------------------------------------------------------------------
# Linear, RMSNorm, argmax known answers
# --------------------------------------------------------------------------

def test_dense_linear_hand_product(orc):
    """linear.rs:337-351 (bias-free part): [1,1] . [[1,2],[3,4]]^T = [3, 7]."""
    y = orc.linear_dense(np.array([[1, 1]], np.float32), np.array([[1, 2], [3, 4]], np.float32))
    assert y.tolist() == [[3.0, 7.0]]


def test_linear_preserves_leading_dimensions(orc):
    """linear.rs:353-364."""
    y = orc.linear_dense(np.zeros((2, 5, 3), np.float32), np.zeros((7, 3), np.float32))
    assert y.shape == (2, 5, 7)


def test_rmsnorm_closed_form(orc):
    y = orc.rmsnorm(np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32), 0.0)
    r = 1.0 / math.sqrt(12.5)
    assert np.allclose(y, [[3 * r, 8 * r]], rtol=1e-7)
    z = orc.rmsnorm(np.zeros((1, 8), np.float32), np.ones(8, np.float32), 1e-6)
    assert np.all(z == 0)  # zero rows stay exactly zero (pad rows)


def test_argmax_picks_the_largest_logit_per_row(orc):
    """engine.rs:601-615 (2-D form); ties go to the first index."""
    assert orc.argmax_rows(np.array([[0.1, 0.9, 0.2], [5.0, 1.0, 2.0]], np.float32)).tolist() == [1, 0]
    assert orc.argmax_rows(np.array([[1.0, 3.0, 3.0]], np.float32)).tolist() == [1]


def test_text_config_widths(fmd):
    """config.rs:244-264."""
    c = fmd.QWEN3_0_6B
    assert (c.q_dim(), c.kv_dim(), c.kv_repeat()) == (2048, 1024, 2)


# --------------------------------------------------------------------------
# Whole decoder: the C oracle against the independent torch restatement
# --------------------------------------------------------------------------

def _tiny(fmd, layers=2, vocab=512):
    return fmd.TextConfig(vocab_size=vocab, hidden_size=256, intermediate_size=512,
                          num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                          head_dim=128, rope_theta=1e6)


def test_cache_lengths_and_overflow(fmd, orc):
    """qwen3.rs:601-633 restated on the oracle: append advances len; overflow errors."""
    cfg = _tiny(fmd, layers=1)
    w = fmd.synthetic_weights(cfg, seed=0)
    m = orc.OracleModel(cfg, orc.F32, 64).load(w)
    kv = m.new_kv(2, 8)
    assert kv.len() == 0
    emb = np.zeros((2, 3, cfg.hidden_size), np.float32)
    m.prefill(kv, emb, [0, 0])
    assert kv.len() == 3
    m.decode_step(kv, [1, 2], [0, 0])
    assert kv.len() == 4
    small = m.new_kv(1, 4)
    with pytest.raises(orc.OracleError, match="kv cache overflow: 0 \\+ 5 exceeds capacity 4"):
        m.prefill(small, np.zeros((1, 5, cfg.hidden_size), np.float32), [0])


def test_cache_bytes(fmd):
    """qwen3.rs:628-633."""
    assert fmd.KvCache.bytes_per_layer(4, 8, 1000, 128, 2) == 2 * 4 * 8 * 1000 * 128 * 2


@pytest.mark.parametrize("block", [256, 5])
def test_oracle_matches_torch_restatement(fmd, orc, block):
    cfg = _tiny(fmd)
    w = fmd.synthetic_weights(cfg, seed=11)
    m = orc.OracleModel(cfg, orc.F32, 256).load(w)
    from tests.torch_ref import TorchQwen3

    tq = TorchQwen3(cfg, w, max_len=256)
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in (9, 3, 14, 0)]
    eos = 7
    force = [-1, 2, -1, -1]
    got = m.generate(prompts, 6, eos, force, block=block)
    toks, fin, all_logits = tq.generate(prompts, 6, eos, force)
    # logits of the prefill and the first decode steps agree to 1e-4 (fp32)
    emb, pad = m.padded_embeds(prompts)
    kv = m.new_kv(len(prompts), emb.shape[1] + 6)
    lg = m.prefill(kv, emb, pad, block=block)
    assert np.max(np.abs(lg - all_logits[0].numpy())) < 1e-4
    for i, (t, f) in enumerate(got):
        assert t == toks[i] and f == fin[i]


def test_pad_rows_stay_exactly_zero(fmd, orc):
    """Left-pad rows and their K/V are exactly zero in every layer (the
    property that lets the device skip them)."""
    cfg = _tiny(fmd)
    m = orc.OracleModel(cfg, orc.BF16, 64).load(fmd.synthetic_weights(cfg, seed=3))
    prompts = [[5, 6, 7, 8, 9, 10], [11, 12]]
    emb, pad = m.padded_embeds(prompts)
    kv = m.new_kv(2, 8)
    m.prefill(kv, emb, pad, block=4)
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            c = kv.read(layer, which)
            assert np.all(c[1, :, :4] == 0)   # row 1's four pad positions
            assert np.all(c[:, :, 6:] == 0)   # never written
            assert np.any(c[1, :, 4:6] != 0) and np.any(c[0, :, :6] != 0)
