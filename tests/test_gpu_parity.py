"""HIP decoder vs the CPU oracle on the same seeded inputs, through the C ABI.

Bars: Q8_0 bytes and KV-cache indexing bit-exact; logits within 2e-2
(bf16 / f16 / int8) and 1e-4 (f32); greedy tokens equal wherever the
oracle's top-2 margin exceeds that tolerance.
"""
import numpy as np
import pytest
import torch

from tests.gpu_util import (OPREC, TOL, assert_logits_match, build_pair, check_greedy, small_cfg,
                            snapshot_kv, storage_to_f32, tiny_cfg, torch_twin, twin_decode_step)

pytestmark = pytest.mark.gpu

PRECS = ["f32", "f16", "bf16", "int8"]


def _announce(msg):
    print(f"[gpu] {msg}", flush=True)


# --------------------------------------------------------------------------
# load-time: Q8_0 quantisation on the device (bit-exact)
# --------------------------------------------------------------------------

def test_q8_0_device_quantisation_bit_exact(fmd, orc):
    _announce("q8_0 quantisation tiny")
    cfg = tiny_cfg(fmd)
    w = fmd.synthetic_weights(cfg, seed=21)
    # make some blocks hit the special cases: zero, exact scale, ties
    key = "model.language_model.layers.0.self_attn.q_proj.weight"
    w[key][0, :32] = 0.0
    w[key][1, :32] = np.arange(32, dtype=np.float32) - 15.5
    w[key][2, :32] = 0.5
    w[key][2, 0] = 127.0
    gpu = fmd.Qwen3(cfg, "int8", max_len=64).load(w)
    for name, src in w.items():
        if src.ndim != 2:
            continue
        got = gpu.q8_0_blocks(name)
        want = orc.quantize_q8_0(src)
        assert np.array_equal(got, want), name
    # tied lm_head = Q8_0 of the f32 embedding (qwen3.rs:566-572)
    got = gpu.q8_0_blocks("model.language_model.lm_head.weight")
    assert np.array_equal(got, orc.quantize_q8_0(w["model.language_model.embed_tokens.weight"]))


def test_q8_0_full_width_projection_bit_exact(fmd, orc):
    _announce("q8_0 full-width layer")
    cfg = small_cfg(fmd, layers=1, vocab=1024)
    w = fmd.synthetic_weights(cfg, seed=22)
    gpu = fmd.Qwen3(cfg, "int8", max_len=64).load(w)
    for part in ("self_attn.q_proj", "self_attn.v_proj", "mlp.up_proj", "mlp.down_proj"):
        name = f"model.language_model.layers.0.{part}.weight"
        assert np.array_equal(gpu.q8_0_blocks(name), orc.quantize_q8_0(w[name])), name


def test_activation_conversion_bit_exact(fmd, orc):
    """The device's f32 -> bf16 / f16 rounding (the embedding table is
    converted on load and read back by embed) equals IEEE round-to-nearest-
    even on special values: ties, subnormals, overflow, signed zeros."""
    _announce("f32 -> bf16/f16 conversion")
    cfg = tiny_cfg(fmd, layers=1, vocab=64)
    rng = np.random.default_rng(5)
    w = fmd.synthetic_weights(cfg, seed=5)
    E = (rng.standard_normal((cfg.vocab_size, cfg.hidden_size)) *
         np.exp(rng.uniform(-30, 30, (cfg.vocab_size, 1)))).astype(np.float32)
    bits = E.view(np.uint32)
    bits[0, :16] = [0x3f808000, 0x3f818000, 0x3f80c000, 0x00000001, 0x80000001, 0x007fffff,
                    0x7f7fffff, 0xff7fffff, 0x00000000, 0x80000000, 0x7f800000, 0xff800000,
                    0x33800000, 0x33800001, 0x38000000, 0x477fe000]
    w["model.language_model.embed_tokens.weight"] = E
    for prec in ("bf16", "f16"):
        gpu = fmd.Qwen3(cfg, prec, max_len=16).load(w)
        got = gpu.embed(np.arange(cfg.vocab_size))
        want = orc.to_storage(E, OPREC[prec])
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), prec


# --------------------------------------------------------------------------
# single projections
# --------------------------------------------------------------------------

def _op_linear(gpu, prec, layer, proj, x_store):
    dev = torch.device("cuda:0")
    x = torch.from_numpy(np.ascontiguousarray(x_store)).to(dev)
    cfg = gpu.cfg
    out_dim = {0: cfg.q_dim() + 2 * cfg.kv_dim(), 1: cfg.hidden_size,
               2: 2 * cfg.intermediate_size, 3: cfg.hidden_size, 4: cfg.vocab_size}[proj]
    odt = torch.float32 if proj == 4 else {"f32": torch.float32, "f16": torch.float16,
                                            "int8": torch.float16, "bf16": torch.bfloat16}[prec]
    y = torch.empty((x_store.shape[0], out_dim), dtype=odt, device=dev)
    torch.cuda.synchronize()  # x is written on torch's stream; the op runs on the handle's
    gpu.op_linear(layer, proj, x.data_ptr(), x_store.shape[0], y.data_ptr())
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("prec", PRECS)
@pytest.mark.parametrize("rows", [1, 8, 16, 37])
def test_linear_projections(fmd, orc, prec, rows):
    _announce(f"linear {prec} rows={rows}")
    cfg = tiny_cfg(fmd, layers=1)
    gpu, ref, w = build_pair(fmd, orc, cfg, prec, seed=31, max_len=64)
    rng = np.random.default_rng(rows)
    P = "model.language_model."
    srcs = {
        0: np.concatenate([w[P + "layers.0.self_attn.q_proj.weight"], w[P + "layers.0.self_attn.k_proj.weight"],
                           w[P + "layers.0.self_attn.v_proj.weight"]]),
        1: w[P + "layers.0.self_attn.o_proj.weight"],
        2: np.concatenate([w[P + "layers.0.mlp.gate_proj.weight"], w[P + "layers.0.mlp.up_proj.weight"]]),
        3: w[P + "layers.0.mlp.down_proj.weight"],
        4: w[P + "embed_tokens.weight"],
    }
    for proj, W in srcs.items():
        if proj == 4 and rows > 16:
            continue
        x = orc.round_to(rng.standard_normal((rows, W.shape[1])).astype(np.float32), OPREC[prec])
        xs = orc.to_storage(x, OPREC[prec])
        got = _op_linear(gpu, prec, 0, proj, xs)
        if prec == "int8":
            want = orc.linear_q8_0(x, orc.quantize_q8_0(W), W.shape[0], OPREC[prec])
        else:
            want = orc.linear_dense(x, orc.round_to(W, OPREC[prec]), OPREC[prec])
        # both round an f32 sum (different orders) to the dtype: one dtype ulp
        # plus f32 reassociation noise relative to sum |x||w|
        ulp = {"f32": 0.0, "f16": 2**-10, "int8": 2**-10, "bf16": 2**-7}[prec]
        Wd = orc.dequantize_q8_0(orc.quantize_q8_0(W), *W.shape) if prec == "int8" else W
        scale = np.abs(x) @ np.abs(Wd).T
        tol = ulp * np.abs(want) + 1e-6 * scale + 1e-7
        assert np.all(np.abs(got - want) <= tol), (proj, np.max(np.abs(got - want) - tol))


@pytest.mark.parametrize("prec,rows", [("bf16", 130), ("bf16", 2100), ("bf16", 4000),
                                       ("int8", 130), ("int8", 2100)])
def test_linear_projections_gemm_tiles(fmd, orc, prec, rows):
    """Prefill GEMM at full widths: ragged last row tiles, the padded XCD
    blocks of every projection shape, and for bf16 each tile kind: 130 rows
    64-row register-staged (O, down) and 128-row (qkv, gate|up) tiles, 2100
    rows 64-row direct-to-LDS (O, down) and 128-row tiles, 4000 rows 256-row
    (qkv, gate|up) tiles."""
    _announce(f"gemm tiles {prec} rows={rows}")
    cfg = small_cfg(fmd, layers=1, vocab=256)
    gpu, ref, w = build_pair(fmd, orc, cfg, prec, seed=33, max_len=64)
    rng = np.random.default_rng(rows + 1)
    P = "model.language_model."
    srcs = {
        0: np.concatenate([w[P + "layers.0.self_attn.q_proj.weight"], w[P + "layers.0.self_attn.k_proj.weight"],
                           w[P + "layers.0.self_attn.v_proj.weight"]]),
        1: w[P + "layers.0.self_attn.o_proj.weight"],
        2: np.concatenate([w[P + "layers.0.mlp.gate_proj.weight"], w[P + "layers.0.mlp.up_proj.weight"]]),
        3: w[P + "layers.0.mlp.down_proj.weight"],
    }
    for proj, W in srcs.items():
        x = orc.round_to(rng.standard_normal((rows, W.shape[1])).astype(np.float32), OPREC[prec])
        got = _op_linear(gpu, prec, 0, proj, orc.to_storage(x, OPREC[prec]))
        if prec == "int8":
            want = orc.linear_q8_0(x, orc.quantize_q8_0(W), W.shape[0], OPREC[prec])
        else:
            want = orc.linear_dense(x, orc.round_to(W, OPREC[prec]), OPREC[prec])
        ulp = {"int8": 2**-10, "bf16": 2**-7}[prec]
        Wd = orc.dequantize_q8_0(orc.quantize_q8_0(W), *W.shape) if prec == "int8" else W
        tol = ulp * np.abs(want) + 1e-6 * (np.abs(x) @ np.abs(Wd).T) + 1e-7
        assert np.all(np.abs(got - want) <= tol), (proj, np.max(np.abs(got - want) - tol))


# --------------------------------------------------------------------------
# decode step over a synthetic padded context (configs 2 / 3 style)
# --------------------------------------------------------------------------

def _synthetic_context(gpu, ref, orc, prec, B, ctx_lens, cap, seed):
    """Same random K/V (rounded to the dtype) in both caches; len = max ctx."""
    cfg = gpu.cfg
    L = max(ctx_lens)
    pad = np.array([L - c for c in ctx_lens], dtype=np.int32)
    gkv = gpu.new_caches(B, cap)
    rkv = ref.new_kv(B, cap)
    rng = np.random.default_rng(seed)
    shape = (B, cfg.num_key_value_heads, cap, cfg.head_dim)
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            x = np.zeros(shape, dtype=np.float32)
            for b in range(B):
                x[b, :, pad[b]:L] = rng.standard_normal((cfg.num_key_value_heads, L - pad[b], cfg.head_dim))
            x = orc.round_to(x, OPREC[prec])
            rkv.write(layer, which, x)
            gkv.write(layer, which, orc.to_storage(x, OPREC[prec]))
    rkv.set_len(L)
    gkv.set_len(L)
    return gkv, rkv, pad


@pytest.mark.parametrize("prec", PRECS)
def test_decode_step_tiny(fmd, orc, prec):
    _announce(f"decode step tiny {prec}")
    cfg = tiny_cfg(fmd)
    gpu, ref, _ = build_pair(fmd, orc, cfg, prec, seed=41, max_len=2048)
    B = 5
    gkv, rkv, pad = _synthetic_context(gpu, ref, orc, prec, B, [300, 17, 1, 299, 64], 400, seed=42)
    ids = [3, 99, 511, 0, 1023]
    for step in range(3):
        g = gpu.decode_step(ids, gkv, pad)
        r = ref.decode_step(rkv, ids, pad)
        assert_logits_match(g, r, prec, what=f"tiny decode step {step}")
        ids = [int(v) for v in r.argmax(-1)]
    assert gkv.len() == rkv.len() == 303


@pytest.mark.parametrize("prec,B", [("int8", 8), ("bf16", 8), ("int8", 16)])
def test_decode_step_full_width(fmd, orc, prec, B):
    """Full layer widths (hidden 1024, 16/8 heads, FFN 3072), contexts 1-3k."""
    _announce(f"decode step full width {prec} B={B}")
    cfg = small_cfg(fmd)
    gpu, ref, w = build_pair(fmd, orc, cfg, prec, seed=51, max_len=4096)
    rng = np.random.default_rng(52)
    lens = rng.integers(1024, 3000, B).tolist()
    gkv, rkv, pad = _synthetic_context(gpu, ref, orc, prec, B, lens, max(lens) + 4, seed=53)
    ids = rng.integers(0, cfg.vocab_size, B).tolist()
    snap = snapshot_kv(rkv, cfg.num_hidden_layers)
    g = gpu.decode_step(ids, gkv, pad)
    r = ref.decode_step(rkv, ids, pad)
    t = twin_decode_step(torch_twin(orc, cfg, w, prec, 4096), snap, ids, pad, max(lens))
    assert_logits_match(g, r, prec, twin=t, what=f"full-width decode B={B}")
    # the new token's K/V landed at position max(lens) of every row
    L = max(lens)
    for which in (0, 1):
        gk = storage_to_f32(gkv.read(0, which), prec)
        rk = rkv.read(0, which)
        assert np.max(np.abs(gk[:, :, L] - rk[:, :, L])) < 0.05
        assert np.array_equal(gk[:, :, L + 1:], rk[:, :, L + 1:])  # untouched zeros


def _oracle_attention_step(orc, cfg, prec, w, qkv, K, V, pad, pos):
    """Reference decode attention of one layer for raw qkv rows: q/k RMSNorm
    over head_dim, RoPE at `pos`, append at `pos`, attend [pad_b, pos]
    (qwen3.rs:213-257) -- composed from the oracle's single ops."""
    P = "model.language_model.layers.0.self_attn."
    B = qkv.shape[0]
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    pr = OPREC[prec]
    q = orc.rmsnorm(qkv[:, : nh * hd].reshape(B, nh, hd), orc.round_to(w[P + "q_norm.weight"], pr),
                    cfg.rms_norm_eps, pr)
    k = orc.rmsnorm(qkv[:, nh * hd: (nh + nkv) * hd].reshape(B, nkv, hd),
                    orc.round_to(w[P + "k_norm.weight"], pr), cfg.rms_norm_eps, pr)
    v = qkv[:, (nh + nkv) * hd:].reshape(B, nkv, hd)
    c, s_ = orc.rope_tables(hd, cfg.rope_theta, pos + 1, pr)
    q = orc.rope_apply(q[:, :, None], pos, c, s_, pr)
    k = orc.rope_apply(k[:, :, None], pos, c, s_, pr)[:, :, 0]
    K = K.copy(); V = V.copy()
    K[:, :, pos] = k
    V[:, :, pos] = v
    mask = orc.build_mask(B, nh // nkv, pos, 1, pos + 1, pad)
    return orc.attention(q, K, V, mask, pos + 1, pr)[:, 0], K, V


@pytest.mark.parametrize("prec,B,lo,hi", [("bf16", 8, 2048, 6144), ("int8", 8, 1024, 4096),
                                          ("int8", 16, 1024, 4096), ("f32", 3, 1, 700),
                                          ("bf16", 4, 14000, 20000), ("int8", 2, 30000, 40000)])
def test_attention_decode_op(fmd, orc, prec, B, lo, hi):
    """Decode attention alone at the configs' shapes (16/8 heads, hd 128):
    ragged valid lengths U[lo, hi], left-padded cache, K/V ~ N(0,1), raw
    q/k/v ~ N(0,1); context within the logits tolerance and the appended K/V
    at the right slots.  The two long-context cases take 512 and 1024 keys
    per work-group (a unit holds at most 64 splits)."""
    _announce(f"attention op {prec} B={B} [{lo},{hi}]")
    cfg = small_cfg(fmd, layers=1, vocab=256)
    w = fmd.synthetic_weights(cfg, seed=33)
    gpu = fmd.Qwen3(cfg, prec, max_len=hi + 8).load(w)
    rng = np.random.default_rng(34)
    lens = rng.integers(lo, hi + 1, B)
    pos = int(lens.max())
    pad = (pos - lens).astype(np.int32)
    cap = pos + 4
    kv = gpu.new_caches(B, cap)
    pr = OPREC[prec]
    shape = kv.shape()
    KV = []
    for which in (0, 1):
        x = np.zeros(shape, dtype=np.float32)
        for b in range(B):
            x[b, :, pad[b]:pos] = rng.standard_normal((shape[1], pos - pad[b], shape[3]))
        x = orc.round_to(x, pr)
        kv.write(0, which, orc.to_storage(x, pr))
        KV.append(x)
    kv.set_len(pos)
    qkv = orc.round_to(rng.standard_normal((B, cfg.q_dim() + 2 * cfg.kv_dim())).astype(np.float32), pr)
    dqkv = torch.from_numpy(orc.to_storage(qkv, pr).copy()).cuda()
    odt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16, "int8": torch.float16}[prec]
    out = torch.empty(B, cfg.q_dim(), dtype=odt, device="cuda")
    torch.cuda.synchronize()  # qkv is written on torch's stream; the op runs on the handle's
    gpu.op_attention_decode(kv, 0, dqkv.data_ptr(), pad, B, out.data_ptr())
    torch.cuda.synchronize()
    want, K2, V2 = _oracle_attention_step(orc, cfg, prec, w, qkv, KV[0], KV[1], pad, pos)
    got = out.float().cpu().numpy()
    assert np.max(np.abs(got - want)) < TOL[prec], np.max(np.abs(got - want))
    assert kv.len() == pos
    gk = storage_to_f32(kv.read(0, 0), prec)
    gv = storage_to_f32(kv.read(0, 1), prec)
    assert np.array_equal(gv, V2)            # v stored as projected: exact
    assert np.max(np.abs(gk - K2)) <= (1e-6 if prec == "f32" else 2 ** -7)
    assert np.array_equal(gk[:, :, :pos], K2[:, :, :pos])  # nothing else touched


def test_attention_exchange_buffers_regrow_across_handles(fmd, orc):
    """A handle's exchange buffers grow with the batch, and a regrown buffer
    can land on memory another (destroyed) handle used, at the same address,
    holding words whose epochs collide with the new handle's (every handle
    counts its launches from 1).  Two handles in turn, each at a larger then
    a smaller-but-wider plan, every context against the oracle."""
    _announce("attention exchange buffers across handles")
    cfg = small_cfg(fmd, layers=1, vocab=256)
    w = fmd.synthetic_weights(cfg, seed=35)
    for prec in ("int8", "bf16"):
        gpu = fmd.Qwen3(cfg, prec, max_len=4096).load(w)
        pr = OPREC[prec]
        for B, lo, hi, seed in ((12, 1000, 3000, 36), (5, 233, 700, 37)):
            rng = np.random.default_rng(seed)
            lens = rng.integers(lo, hi + 1, B)
            pos = int(lens.max())
            pad = (pos - lens).astype(np.int32)
            kv = gpu.new_caches(B, pos + 4)
            KV = []
            for which in (0, 1):
                x = orc.round_to(rng.standard_normal(kv.shape()).astype(np.float32), pr)
                kv.write(0, which, orc.to_storage(x, pr))
                KV.append(x)
            kv.set_len(pos)
            qkv = orc.round_to(rng.standard_normal((B, cfg.q_dim() + 2 * cfg.kv_dim())).astype(np.float32), pr)
            dqkv = torch.from_numpy(orc.to_storage(qkv, pr).copy()).cuda()
            odt = torch.bfloat16 if prec == "bf16" else torch.float16
            out = torch.empty(B, cfg.q_dim(), dtype=odt, device="cuda")
            torch.cuda.synchronize()
            gpu.op_attention_decode(kv, 0, dqkv.data_ptr(), pad, B, out.data_ptr())
            torch.cuda.synchronize()
            want, _, _ = _oracle_attention_step(orc, cfg, prec, w, qkv, KV[0], KV[1], pad, pos)
            d = float(np.max(np.abs(out.float().cpu().numpy() - want)))
            assert d < TOL[prec], (prec, B, d)
        del gpu, kv


# --------------------------------------------------------------------------
# prefill + KV-cache contents
# --------------------------------------------------------------------------

@pytest.mark.parametrize("prec", PRECS)
@pytest.mark.parametrize("chunk", [256, 64])
def test_prefill_logits_and_cache(fmd, orc, prec, chunk):
    _announce(f"prefill {prec} chunk={chunk}")
    cfg = tiny_cfg(fmd)
    gpu, ref, w = build_pair(fmd, orc, cfg, prec, seed=61, max_len=2048)
    rng = np.random.default_rng(62)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in (300, 41, 1, 257, 0, 128)]
    emb, pad = ref.padded_embeds(prompts)
    B, T = len(prompts), emb.shape[1]
    gkv = gpu.new_caches(B, T + 8)
    rkv = ref.new_kv(B, T + 8)
    g = gpu.prefill(orc.to_storage(emb, OPREC[prec]), gkv, pad, chunk=chunk)
    r = ref.prefill(rkv, emb, pad, block=256)
    twin = torch_twin(orc, cfg, w, prec, T + 8)
    zeros = [torch.zeros(B, cfg.num_key_value_heads, T + 8, cfg.head_dim)
             for _ in range(cfg.num_hidden_layers)]
    t = twin.forward(torch.from_numpy(emb), zeros, [z.clone() for z in zeros], 0,
                     [int(x) for x in pad]).numpy()
    assert_logits_match(g, r, prec, twin=t, what=f"prefill chunk={chunk}")
    assert gkv.len() == T
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            gk = storage_to_f32(gkv.read(layer, which), prec)
            rk = rkv.read(layer, which)
            real = np.zeros(gk.shape, dtype=bool)
            for b in range(B):
                real[b, :, pad[b]:T] = True
            # pad and unwritten slots are exactly zero on both sides
            assert np.all(gk[~real] == 0) and np.all(rk[~real] == 0)
            tol = 1e-3 if prec == "f32" else 0.1
            assert np.max(np.abs(gk[real] - rk[real])) < tol, (layer, which)


@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (8, 2)])
@pytest.mark.parametrize("chunk", [256, 64])
def test_prefill_gqa_repeats(fmd, orc, heads, kv_heads, chunk):
    """Prefill attention at GQA repeats 1 and 4 (the model runs at 2), bf16:
    one-launch tiles (short key ranges) and split tiles (more than 256 keys)
    against the oracle, logits and cache."""
    _announce(f"prefill bf16 heads={heads} kv={kv_heads} chunk={chunk}")
    cfg = fmd.TextConfig(vocab_size=1024, hidden_size=256, intermediate_size=512,
                         num_hidden_layers=2, num_attention_heads=heads,
                         num_key_value_heads=kv_heads, head_dim=128, rope_theta=1e6)
    prec = "bf16"
    gpu, ref, w = build_pair(fmd, orc, cfg, prec, seed=67, max_len=2048)
    rng = np.random.default_rng(68)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in (300, 41, 1, 257, 0, 128)]
    emb, pad = ref.padded_embeds(prompts)
    B, T = len(prompts), emb.shape[1]
    gkv = gpu.new_caches(B, T + 8)
    rkv = ref.new_kv(B, T + 8)
    g = gpu.prefill(orc.to_storage(emb, OPREC[prec]), gkv, pad, chunk=chunk)
    r = ref.prefill(rkv, emb, pad, block=256)
    twin = torch_twin(orc, cfg, w, prec, T + 8)
    zeros = [torch.zeros(B, cfg.num_key_value_heads, T + 8, cfg.head_dim)
             for _ in range(cfg.num_hidden_layers)]
    t = twin.forward(torch.from_numpy(emb), zeros, [z.clone() for z in zeros], 0,
                     [int(x) for x in pad]).numpy()
    assert_logits_match(g, r, prec, twin=t, what=f"prefill rep={heads // kv_heads} chunk={chunk}")
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            gk = storage_to_f32(gkv.read(layer, which), prec)
            rk = rkv.read(layer, which)
            real = np.zeros(gk.shape, dtype=bool)
            for b in range(B):
                real[b, :, pad[b]:T] = True
            assert np.all(gk[~real] == 0) and np.all(rk[~real] == 0)
            assert np.max(np.abs(gk[real] - rk[real])) < 0.1, (layer, which)


def _selection_model(fmd, seed, heads=4, kv_heads=2):
    """A configuration whose layer-0 K and V are exact functions of the token
    ids, so any two correct implementations store identical bits: embedding
    entries are +-1 and the gains 1 (so the RMSNorm scale is exactly 1 with
    eps = 2^-30), and each k/v output copies one input element times 127/128
    (exact in Q8_0 too: d = 2^-7, q = 127), whose squares sum exactly in any
    order."""
    cfg = tiny_cfg(fmd)
    cfg.num_attention_heads, cfg.num_key_value_heads = heads, kv_heads
    cfg.rms_norm_eps = 2.0**-30
    w = fmd.synthetic_weights(cfg, seed=seed)
    P = "model.language_model."
    rng = np.random.default_rng(seed)
    H = cfg.hidden_size
    for part in ("k_proj", "v_proj"):
        sel = np.zeros((cfg.kv_dim(), H), dtype=np.float32)
        sel[np.arange(cfg.kv_dim()), rng.integers(0, H, cfg.kv_dim())] = 127.0 / 128.0
        w[P + f"layers.0.self_attn.{part}.weight"] = sel
    w[P + "layers.0.input_layernorm.weight"] = np.ones(H, np.float32)
    w[P + "layers.0.self_attn.k_norm.weight"] = np.ones(cfg.head_dim, np.float32)
    w[P + "embed_tokens.weight"] = rng.choice(np.array([-1.0, 1.0], np.float32), (cfg.vocab_size, H))
    return cfg, w


@pytest.mark.parametrize("prec", ["f32", "bf16", "int8"])
def test_kv_cache_indexing_bit_exact(fmd, orc, prec):
    """Layer-0 K and V after prefill + decode steps are bit-identical to the
    oracle's at every (row, head, position, dim), pads and unwritten slots
    included (KvCache::append, qwen3.rs:86-101; pad/offset engine.rs:470-533)."""
    _announce(f"kv indexing {prec}")
    cfg, w = _selection_model(fmd, seed=71)
    gpu, ref, _ = build_pair(fmd, orc, cfg, prec, weights=w, max_len=1024)
    rng = np.random.default_rng(72)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in (70, 3, 129, 1)]
    emb, pad = ref.padded_embeds(prompts)
    B, T = len(prompts), emb.shape[1]
    gkv = gpu.new_caches(B, T + 6)
    rkv = ref.new_kv(B, T + 6)
    gpu.prefill(orc.to_storage(emb, OPREC[prec]), gkv, pad, chunk=64)
    ref.prefill(rkv, emb, pad)
    for step in range(3):
        ids = rng.integers(0, cfg.vocab_size, B).tolist()
        gpu.decode_step(ids, gkv, pad)
        ref.decode_step(rkv, ids, pad)
    real = np.zeros(gkv.shape(), dtype=bool)
    for b in range(B):
        real[b, :, pad[b]:T + 3] = True
    for which in (0, 1):
        g = gkv.read(0, which)
        r = orc.to_storage(rkv.read(0, which), OPREC[prec])
        # written positions: identical bits
        gb = g.view(np.uint16 if g.itemsize == 2 else np.uint32)
        rb = r.view(np.uint16 if r.itemsize == 2 else np.uint32)
        assert np.array_equal(gb[real], rb[real]), which
        # pad and unwritten slots: exactly zero (the reference computes pad rows,
        # whose RoPE can leave -0.0; the sign of those never-read zeros is unpinned)
        gz = storage_to_f32(g, prec)[~real]
        rz = storage_to_f32(r, prec)[~real]
        assert np.all(gz == 0) and np.all(rz == 0), which
        assert np.count_nonzero(gb[real]) > real.sum() // 2  # the check is not vacuous


@pytest.mark.parametrize("prec", ["bf16", "f16"])
@pytest.mark.parametrize("heads,kv_heads,lens,chunk", [
    # 8 column groups of q|k|v: the 2460-row first chunk takes the 64-row
    # direct-to-LDS tiles, the 940-row second chunk the register-staged ones
    (4, 2, (700, 690, 680, 670, 660), 512),
    # 16 column groups: 128-row tiles at any row count
    (8, 4, (300, 41, 129, 1), 256),
])
def test_kv_cache_bit_exact_across_prefill_tiles(fmd, orc, prec, heads, kv_heads, lens, chunk):
    """The q|k|v projection's fused q/k norm + RoPE + cache-store epilogue in
    each of its tile kinds.  On the selection model, layer-0 K and V after
    prefill are bit-identical to the oracle's (qwen3.rs:213-227 then
    KvCache::append, qwen3.rs:86-101) and pads exactly zero; with the usual
    N(0, 0.02) weights the logits (which the q path feeds) agree with the
    oracle's."""
    _announce(f"kv bit-exact {prec} heads={heads}/{kv_heads} lens={lens} chunk={chunk}")
    cfg, w = _selection_model(fmd, seed=73, heads=heads, kv_heads=kv_heads)
    gpu, ref, _ = build_pair(fmd, orc, cfg, prec, weights=w, max_len=1024)
    rng = np.random.default_rng(74)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    emb, pad = ref.padded_embeds(prompts)
    B, T = len(prompts), emb.shape[1]
    gkv = gpu.new_caches(B, T + 2)
    rkv = ref.new_kv(B, T + 2)
    gpu.prefill(orc.to_storage(emb, OPREC[prec]), gkv, pad, chunk=chunk)
    ref.prefill(rkv, emb, pad)
    real = np.zeros(gkv.shape(), dtype=bool)
    for b in range(B):
        real[b, :, pad[b]:T] = True
    for which in (0, 1):
        gb = gkv.read(0, which).view(np.uint16)
        rb = orc.to_storage(rkv.read(0, which), OPREC[prec]).view(np.uint16)
        assert np.array_equal(gb[real], rb[real]), which
        assert np.all(storage_to_f32(gkv.read(0, which), prec)[~real] == 0), which
        assert np.count_nonzero(gb[real]) > real.sum() // 2
    del gpu, ref, gkv, rkv
    # the same shapes with the usual weights: logits
    cfg2 = tiny_cfg(fmd)
    cfg2.num_attention_heads, cfg2.num_key_value_heads = heads, kv_heads
    gpu, ref, w2 = build_pair(fmd, orc, cfg2, prec, seed=75, max_len=1024)
    emb, pad = ref.padded_embeds(prompts)
    g = gpu.prefill(orc.to_storage(emb, OPREC[prec]), gpu.new_caches(B, T + 2), pad, chunk=chunk)
    r = ref.prefill(ref.new_kv(B, T + 2), emb, pad)
    twin = torch_twin(orc, cfg2, w2, prec, T + 2)
    zeros = [torch.zeros(B, cfg2.num_key_value_heads, T + 2, cfg2.head_dim)
             for _ in range(cfg2.num_hidden_layers)]
    t = twin.forward(torch.from_numpy(emb), zeros, [z.clone() for z in zeros], 0,
                     [int(x) for x in pad]).numpy()
    assert_logits_match(g, r, prec, twin=t, what=f"prefill tiles heads={heads}")


# --------------------------------------------------------------------------
# greedy generation (engine.rs:463-541)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("prec", PRECS)
def test_generate_matches_oracle(fmd, orc, prec):
    _announce(f"generate {prec}")
    cfg = tiny_cfg(fmd)
    gpu, ref, _ = build_pair(fmd, orc, cfg, prec, seed=81, max_len=2048)
    rng = np.random.default_rng(82)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in (40, 7, 90, 1, 33)]
    eos = int(rng.integers(0, cfg.vocab_size))
    budget = 24
    force = [-1, 5, -1, 0, 30]
    out = gpu.generate_batch(prompts, budget, eos=eos, force_eot_step=force)
    gpu_out = [(o.tokens, int(o.finish_reason)) for o in out]
    n = check_greedy(gpu_out, ref, prompts, budget, eos, TOL[prec], force=force)
    assert n >= 40
    assert gpu_out[1][1] == 1 and len(gpu_out[1][0]) <= 5   # forced end-of-turn at step 5
    assert gpu_out[3] == ([], 1)                             # forced at step 0


def test_host_loop_with_device_greedy_matches_device_loop(fmd, orc):
    """A host-side loop (prefill, then decode_step + fmd_dec_greedy per step,
    as engine.rs:505-537 drives it) yields the same tokens and finish
    reasons as the device loop of fmd_dec_generate, forced end-of-turn
    included."""
    _announce("host loop with device greedy")
    cfg = tiny_cfg(fmd)
    gpu, ref, _ = build_pair(fmd, orc, cfg, "int8", seed=81, max_len=512)
    rng = np.random.default_rng(82)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in (40, 7, 23)]
    budget, eos, force = 12, 5, [-1, 3, -1]
    want = gpu.generate_batch(prompts, budget, eos=eos, force_eot_step=force)
    emb, pad = ref.padded_embeds(prompts)
    B, T = len(prompts), emb.shape[1]
    kv = gpu.new_caches(B, T + budget)
    gpu.prefill(orc.to_storage(emb, OPREC["int8"]), kv, pad, chunk=256)
    done = np.zeros(B, dtype=np.int32)
    toks = [[] for _ in range(B)]
    for step in range(budget):
        nxt, emitted = gpu.greedy(B, step, done, eos=eos, force_eot_step=force)
        for b in range(B):
            if emitted[b] >= 0:
                toks[b].append(emitted[b])
        if done.all() or step + 1 == budget:
            break
        gpu.decode_step(nxt, kv, pad)
    for b in range(B):
        assert toks[b] == want[b].tokens, b
        assert int(done[b]) == int(want[b].finish_reason), b


def test_batched_equals_solo(fmd, orc):
    """python/tests/test_engine.py:148-173 made exact: a row's greedy tokens
    do not depend on its batch-mates (same left padding)."""
    _announce("batched vs solo")
    cfg = tiny_cfg(fmd)
    gpu, _, _ = build_pair(fmd, orc, cfg, "int8", seed=91, max_len=1024)
    rng = np.random.default_rng(92)
    prompts = [rng.integers(0, cfg.vocab_size, 50).tolist() for _ in range(4)]
    batched = gpu.generate_batch(prompts, 16, eos=5)
    for i, p in enumerate(prompts):
        solo = gpu.generate_batch([p], 16, eos=5)[0]
        assert solo.tokens == batched[i].tokens


def test_engine_sorts_and_chunks(fmd, orc):
    """engine.rs:382-424: outputs come back in request order; each micro-batch
    equals generate_batch on its sorted members."""
    _announce("engine")
    cfg = tiny_cfg(fmd)
    gpu, _, _ = build_pair(fmd, orc, cfg, "bf16", seed=93, max_len=1024)
    rng = np.random.default_rng(94)
    lens = [30, 5, 64, 12, 12, 80, 1]
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    eng = fmd.Engine(gpu, fmd.EngineConfig(max_new_tokens=10, max_batch_size=3, eos_id=7))
    res, stats = eng.generate(prompts)
    assert stats.micro_batches == 3
    order = sorted(range(len(lens)), key=lambda i: lens[i])
    for g0 in range(0, len(order), 3):
        group = order[g0:g0 + 3]
        want = gpu.generate_batch([prompts[i] for i in group], 10, eos=7)
        for j, i in enumerate(group):
            assert res[i].tokens == want[j].tokens and res[i].error is None
            assert res[i].prompt_tokens == lens[i]
    assert stats.generated_tokens == sum(len(r.tokens) for r in res)


def test_errors_and_edge_cases(fmd, orc):
    _announce("errors")
    cfg = tiny_cfg(fmd, layers=1)
    gpu, ref, _ = build_pair(fmd, orc, cfg, "bf16", seed=95, max_len=256)
    kv = gpu.new_caches(2, 8)
    with pytest.raises(fmd.KvCacheOverflow, match="kv cache overflow: 0 \\+ 9 exceeds capacity 8"):
        gpu.prefill(np.zeros((2, 9, cfg.hidden_size), np.uint16), kv, [0, 0])
    gpu.prefill(np.zeros((2, 8, cfg.hidden_size), np.uint16), kv, [0, 3])
    with pytest.raises(fmd.KvCacheOverflow):
        gpu.decode_step([1, 2], kv, [0, 3])
    with pytest.raises(fmd.FmdError, match="empty prompt"):
        gpu.generate_batch([[], []], 4, eos=1)
    # budget 1: exactly one greedy pick, no decode step (engine.rs:521-523)
    out = gpu.generate_batch([[1, 2, 3]], 1, eos=999)
    with pytest.raises(fmd.FmdError, match="eos id"):
        gpu.generate_batch([[1, 2, 3]], 4, eos=cfg.vocab_size)
    assert len(out[0].tokens) <= 1
    # truncate keeps the minimum (qwen3.rs:105-107)
    kv.truncate(100)
    assert kv.len() == 8
    kv.truncate(3)
    assert kv.len() == 3
