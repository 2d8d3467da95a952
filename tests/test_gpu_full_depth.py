"""The full Qwen3-0.6B decoder shape (28 layers, hidden 1024, 16/8 heads,
FFN 3072, vocab 151936) on the device, through the C ABI.

- Against the oracle (and the torch twin, which measures the fp32
  summation-order floor): one decode step at batch 8 (bf16, int8) and 16
  (int8) over ragged contexts short enough for the CPU side.
- The benchmark's own shape whole: int8, batch 8, every row 4096 keys, one
  decode step against the oracle at the 2e-2 bar with no twin.
- At the workload sizes of the benchmarks (contexts up to 6144 positions),
  size-independent properties: runs are bit-for-bit deterministic and the
  rows of a batch are independent (a permuted batch gives permuted logits
  and tokens, bit for bit).
"""
import numpy as np
import pytest

from tests.gpu_util import (OPREC, assert_greedy_match, assert_logits_match, snapshot_kv,
                            torch_twin, twin_decode_step)

pytestmark = pytest.mark.gpu


def _announce(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def full_weights(fmd):
    return fmd.synthetic_weights(fmd.QWEN3_0_6B, seed=7)


@pytest.mark.parametrize("prec,B", [("int8", 8), ("int8", 16), ("bf16", 8)])
def test_full_depth_decode_step_vs_oracle(fmd, orc, full_weights, prec, B):
    _announce(f"full depth decode step {prec} B={B}")
    cfg = fmd.QWEN3_0_6B
    rng = np.random.default_rng(100 + B)
    lens = rng.integers(256, 769, B)
    L = int(lens.max())
    pad = (L - lens).astype(np.int32)
    ref = orc.OracleModel(cfg, OPREC[prec], L + 8).load(full_weights)
    rkv = ref.new_kv(B, L + 4)
    rkv.fill_random(9, L)
    gpu = fmd.Qwen3(cfg, prec, max_len=L + 8).load(full_weights)
    gkv = gpu.new_caches(B, L + 4)
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            gkv.write(layer, which, orc.to_storage(rkv.read(layer, which), OPREC[prec]))
    gkv.set_len(L)
    snap = snapshot_kv(rkv, cfg.num_hidden_layers)
    ids = rng.integers(0, cfg.vocab_size, B).tolist()
    g = gpu.decode_step(ids, gkv, pad)
    r = ref.decode_step(rkv, ids, pad)
    del ref
    t = twin_decode_step(torch_twin(orc, cfg, full_weights, prec, L + 8), snap, ids, pad, L)
    assert_logits_match(g, r, prec, twin=t, what=f"full depth B={B}")
    assert_greedy_match(g, r, prec, twin=t)


def test_headline_shape_decode_step_vs_oracle(fmd, orc, full_weights):
    """The benchmark's own shape compared whole: int8 (Q8_0 weights, f16
    activations and cache), batch 8, every row 4096 keys of context, 28
    layers, vocabulary 151936.  One decode step against the oracle on the same
    cache contents, at the 2e-2 bar with no twin; greedy ids equal wherever
    the oracle's top-2 margin exceeds the bar."""
    _announce("headline shape decode step int8 B=8 ctx 4096 vs oracle")
    cfg = fmd.QWEN3_0_6B
    B, L = 8, 4096
    gpu = fmd.Qwen3(cfg, "int8", max_len=L + 8).load(full_weights)
    gkv = gpu.new_caches(B, L + 4)
    gkv.fill_random(13, L)
    ref = orc.OracleModel(cfg, OPREC["int8"], L + 8).load(full_weights)
    rkv = ref.new_kv(B, L + 4)
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            rkv.write(layer, which, gkv.read(layer, which).astype(np.float32))
    rkv.set_len(L)
    ids = np.random.default_rng(14).integers(0, cfg.vocab_size, B).tolist()
    pad = [0] * B
    g = gpu.decode_step(ids, gkv, pad)
    r = ref.decode_step(rkv, ids, pad)
    # the new token's K/V rows, appended at position 4096 of every row: layer
    # 0 (same input) at the bar; the last layer's distance is reported
    for layer in (0, cfg.num_hidden_layers - 1):
        for which in (0, 1):
            d = np.abs(gkv.read(layer, which)[:, :, L].astype(np.float32) -
                       rkv.read(layer, which)[:, :, L])
            print(f"[gap] new {'KV'[which]} row layer {layer}: max {float(d.max()):.4g}", flush=True)
            if layer == 0:
                assert float(d.max()) < 2e-2, (layer, which, float(d.max()))
    del ref, rkv
    assert gkv.len() == L + 1
    assert_logits_match(g, r, "int8", twin=None, what="headline shape B=8 ctx 4096")
    assert_greedy_match(g, r, "int8")


def _copy_rows(cfg, src, dst, rows):
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            dst.write(layer, which, np.ascontiguousarray(src.read(layer, which)[rows]))


@pytest.mark.parametrize("prec,B,lo,hi", [("bf16", 8, 2048, 6144), ("int8", 8, 1024, 4096),
                                          ("int8", 16, 1024, 4096)])
def test_full_size_rows_are_independent(fmd, full_weights, prec, B, lo, hi):
    """At the workload sizes: permuting the rows of a ragged, left-padded
    batch (cache rows, pads and ids together) permutes the logits and the
    greedy tokens bit for bit, and a repeated run is bit-identical."""
    _announce(f"full size row independence {prec} B={B} ctx [{lo},{hi}]")
    cfg = fmd.QWEN3_0_6B
    rng = np.random.default_rng(200 + lo + B)
    lens = rng.integers(lo, hi + 1, B)
    L = int(lens.max())
    pad = (L - lens).astype(np.int32)
    steps = 6
    gpu = fmd.Qwen3(cfg, prec, max_len=L + steps + 8).load(full_weights)
    kv = gpu.new_caches(B, L + steps + 2)
    kv.fill_random(11, L)
    ids = np.asarray(rng.integers(0, cfg.vocab_size, B))
    perm = rng.permutation(B)
    runs = []
    for rows in (np.arange(B), np.arange(B), perm):
        c = gpu.new_caches(B, L + steps + 2)
        _copy_rows(cfg, kv, c, rows)
        c.set_len(L)
        logits = gpu.decode_step(ids[rows].tolist(), c, pad[rows].tolist())
        assert np.all(np.isfinite(logits))
        c.truncate(L)
        gens, _ = gpu.decode_loop(c, ids[rows].tolist(), pad[rows].tolist(), steps, 151645)
        runs.append((logits, [g.tokens for g in gens]))
    assert np.array_equal(runs[0][0], runs[1][0])            # deterministic
    assert runs[0][1] == runs[1][1]
    assert np.array_equal(runs[0][0][perm], runs[2][0])      # rows independent
    assert [runs[0][1][i] for i in perm] == runs[2][1]
    assert all(len(t) > 0 for t in runs[0][1])
