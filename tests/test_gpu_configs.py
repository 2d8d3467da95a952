"""The workload shapes of the benchmark configurations on the HIP path,
against the oracle.

- bf16 chunked prefill at full layer widths (hidden 1024, 16/8 heads, FFN
  3072), 2 layers and a 2048-token vocabulary so the oracle finishes in about
  a minute: 8 prompts with lengths drawn U[1500, 8000] (seed 4), chunk 512 --
  the packed chunks hold thousands of rows, and attention runs its split
  key-range items (about 96 per KV head) and the combine.  Logits within
  2e-2; pad slots exactly zero; layer 0's K and V (computed from the
  embeddings alone) at every valid position within max(2e-2, one bf16 ulp);
  deeper layers' K and V, which carry layer 0's one-ulp output flips through
  attention over thousands of keys (and RoPE moves a flip of a large element
  onto its small partner), within 0.125 everywhere and within 1e-2 relative
  L2 error per (row, KV head).
- fp32, the Qwen3-0.6B shape at full depth and vocabulary: batch 4 with
  prompts {310, 760, 1210, 1890} (seed 1 ids, seed 0 weights), prefill in
  256-position chunks then 32 greedy decode steps; prefill logits within
  1e-4 and greedy ids equal wherever the oracle's top-2 margin exceeds 1e-4.
- int8 end to end at the full shape: 32 requests with prompt lengths
  log-uniform in [500, 8000] (seed 5), micro-batches of 8, up to 1024 new
  tokens with end-of-turn forced at steps U[128, 1024) (seed 6).  Each
  micro-batch of Engine.generate equals generate_batch on its sorted
  members; forced rows stop at their step (or earlier at a natural
  end-of-turn); one micro-batch is replayed through the oracle on a
  2-layer copy of the model.
"""
import numpy as np
import pytest

from tests.gpu_util import OPREC, TOL, check_greedy, small_cfg, storage_to_f32

pytestmark = pytest.mark.gpu

EOS = 151645


def _announce(msg):
    print(f"[gpu] {msg}", flush=True)


def _ulp_bf16(x):
    a = np.maximum(np.abs(x.astype(np.float32)), np.float32(2.0 ** -126))
    return np.exp2(np.floor(np.log2(a)) - 7).astype(np.float32)


@pytest.mark.timeout(900)
def test_bf16_chunked_prefill_full_width_vs_oracle(fmd, orc):
    cfg = small_cfg(fmd, layers=2, vocab=2048)
    rng = np.random.default_rng(4)
    lens = [int(n) for n in rng.integers(1500, 8001, 8)]
    _announce(f"bf16 prefill full width, 2 layers, chunk 512, lengths {lens}")
    w = fmd.synthetic_weights(cfg, seed=41)
    T = max(lens)
    ref = orc.OracleModel(cfg, OPREC["bf16"], T + 8).load(w)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    emb, pad = ref.padded_embeds(prompts)
    gpu = fmd.Qwen3(cfg, "bf16", max_len=T + 8)
    gpu.load(w)
    gkv = gpu.new_caches(8, T + 4)
    got = gpu.prefill(orc.to_storage(emb, OPREC["bf16"]), gkv, pad, chunk=512)
    _announce("device prefill done; oracle prefill (about a minute)")
    rkv = ref.new_kv(8, T + 4)
    want = ref.prefill(rkv, emb, pad, block=256)
    d = np.abs(got - want)
    print(f"[gap] prefill logits max {d.max():.4g} rms {np.sqrt(np.mean(d * d)):.3g}", flush=True)
    assert d.max() < TOL["bf16"], float(d.max())
    for layer in range(cfg.num_hidden_layers):
        for which in (0, 1):
            g = storage_to_f32(gkv.read(layer, which), "bf16")
            r = rkv.read(layer, which)
            worst_rel = 0.0
            for b in range(8):
                p = int(pad[b])
                assert not g[b, :, :p].any() and not g[b, :, T:].any(), (layer, which, b)
                dv = np.abs(g[b, :, p:T] - r[b, :, p:T])
                if layer == 0:
                    # computed from the embeddings alone: one rounding flip at most
                    over1 = dv > np.maximum(TOL["bf16"], _ulp_bf16(r[b, :, p:T]))
                    assert not over1.any(), (layer, which, b, float(dv.max()), int(over1.sum()))
                else:
                    # layer 0's one-ulp output flips reach these rows through
                    # attention over thousands of positions, and RoPE moves a
                    # flip of a large element onto its small partner: sparse
                    # differences of a few large-element ulps, tiny in norm
                    assert dv.max() <= 0.125, (layer, which, b, float(dv.max()))
                    for h in range(cfg.num_key_value_heads):
                        rel = float(np.linalg.norm(dv[h]) / max(np.linalg.norm(r[b, h, p:T]), 1e-30))
                        worst_rel = max(worst_rel, rel)
                        assert rel <= 1e-2, (layer, which, b, h, rel)
            dd = np.abs(g - r)
            print(f"[gap] layer {layer} {'kv'[which]}: max {dd.max():.4g} "
                  f"differing {np.mean(dd > 0):.3%}, worst relative L2 per (row, head) "
                  f"{worst_rel:.3g}", flush=True)


@pytest.mark.timeout(900)
def test_fp32_full_depth_prefill_and_greedy_vs_oracle(fmd, orc):
    cfg = fmd.QWEN3_0_6B
    lens = [310, 760, 1210, 1890]
    _announce(f"fp32 28 layers, batch 4 {lens}: prefill (chunk 256) + 32 greedy steps")
    w = fmd.synthetic_weights(cfg, seed=0)
    rng = np.random.default_rng(1)
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    budget = 33  # greedy step 0 on the prefill logits, then 32 decode steps
    T = max(lens)
    gpu = fmd.Qwen3(cfg, "f32", max_len=T + budget + 8).load(w)
    ref = orc.OracleModel(cfg, OPREC["f32"], T + budget + 8).load(w)
    emb, pad = ref.padded_embeds(prompts)
    gkv = gpu.new_caches(4, T + 4)
    got = gpu.prefill(emb, gkv, pad, chunk=256)
    del gkv
    out = gpu.generate_batch(prompts, budget, eos=EOS, chunk=256)
    _announce("device done; oracle prefill and greedy replay (a minute or two)")
    rkv = ref.new_kv(4, T + 4)
    want = ref.prefill(rkv, emb, pad, block=256)
    del rkv
    d = np.abs(got - want)
    print(f"[gap] fp32 prefill logits max {d.max():.4g}", flush=True)
    assert d.max() < TOL["f32"], float(d.max())
    n = check_greedy([(g.tokens, int(g.finish_reason)) for g in out], ref, prompts, budget, EOS,
                     TOL["f32"])
    print(f"[greedy] fp32 compared {n} tokens", flush=True)
    assert n >= 4 * 16


@pytest.fixture(scope="module")
def e2e_requests(fmd):
    rng = np.random.default_rng(5)
    lens = np.exp(rng.uniform(np.log(500), np.log(8000), 32)).astype(int)
    prompts = [rng.integers(0, fmd.QWEN3_0_6B.vocab_size, int(n)).tolist() for n in lens]
    force = np.random.default_rng(6).integers(128, 1024, 32).tolist()
    return prompts, force


@pytest.mark.timeout(600)
def test_int8_engine_end_to_end_micro_batches(fmd, orc, e2e_requests):
    cfg = fmd.QWEN3_0_6B
    prompts, force = e2e_requests
    budget = 1024
    _announce("int8 e2e: 32 requests, micro-batches of 8, budget 1024, forced EOT")
    w = fmd.synthetic_weights(cfg, seed=0)
    gpu = fmd.Qwen3(cfg, "int8").load(w)
    eng = fmd.Engine(gpu, fmd.EngineConfig(max_new_tokens=budget, max_batch_size=8, eos_id=EOS,
                                           chunk=512))
    res, stats = eng.generate(prompts, force_eot_step=force)
    assert stats.micro_batches == 4
    assert all(r.error is None for r in res)
    assert stats.generated_tokens == sum(len(r.tokens) for r in res)
    order = sorted(range(32), key=lambda i: len(prompts[i]))  # stable, as engine.rs:385
    for m in range(4):
        members = order[8 * m: 8 * m + 8]
        _announce(f"micro-batch {m}: generate_batch on its members")
        alone = gpu.generate_batch([prompts[i] for i in members], budget, eos=EOS,
                                   force_eot_step=[force[i] for i in members], chunk=512)
        for j, i in enumerate(members):
            assert res[i].tokens == alone[j].tokens, (m, i)
            assert res[i].finish_reason == alone[j].finish_reason
    for i in range(32):
        r = res[i]
        assert r.prompt_tokens == len(prompts[i])
        assert len(r.tokens) <= min(budget, force[i])
        assert int(r.finish_reason) == 1  # Stop: forced at a step below the budget
        assert EOS not in r.tokens
    del gpu
    # one micro-batch (the shortest prompts) through the oracle on a 2-layer
    # copy of the same weights, with a short budget and the same forcing rule
    cfg2 = fmd.TextConfig(**{**cfg.__dict__, "num_hidden_layers": 2})
    w2 = {k: v for k, v in w.items() if ".layers." not in k or
          int(k.split(".layers.")[1].split(".")[0]) < 2}
    members = order[:8]
    sub = [prompts[i] for i in members]
    f2 = [7, 30, 3, 30, 12, 30, 30, 1]
    _announce("2-layer copy: one micro-batch against the oracle")
    gpu2 = fmd.Qwen3(cfg2, "int8").load(w2)
    eng2 = fmd.Engine(gpu2, fmd.EngineConfig(max_new_tokens=24, max_batch_size=8, eos_id=EOS,
                                             chunk=512))
    r2, _ = eng2.generate(sub, force_eot_step=f2)
    ref = orc.OracleModel(cfg2, OPREC["int8"], 8192).load(w2)
    n = check_greedy([(r.tokens, int(r.finish_reason)) for r in r2], ref, sub, 24, EOS,
                     TOL["int8"], force=f2)
    print(f"[greedy] int8 2-layer micro-batch compared {n} tokens", flush=True)
    assert n >= 8 * 4
