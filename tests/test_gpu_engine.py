"""Engine semantics of engine.rs:382-424 and the argument checks of the
decode entry points, on the device through the C ABI.

- Micro-batches above 16 rows (max_batch_size has no upper bound in the
  reference, engine.rs:387): a 20-row micro-batch runs as 16-row groups over
  the same padded length; every row's tokens equal the oracle's for the
  whole 20-row batch.
- A failed micro-batch reports "batch generation failed: {e}" against every
  member (engine.rs:414-421), with the library's message.
- Decode positions come from the RoPE table: rows still generating when it
  runs out fail the batch (Rope::apply's narrow, qwen3.rs:139-144); rows
  that all stop before then succeed.
- Pads outside the cache and all-padding prefills are rejected before any
  launch.
"""
import numpy as np
import pytest

from tests.gpu_util import OPREC, TOL, check_greedy, tiny_cfg

pytestmark = pytest.mark.gpu

EOS = 1000


def _announce(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.mark.parametrize("prec", ["int8", "bf16"])
def test_micro_batch_above_16_rows(fmd, orc, prec):
    _announce(f"engine max_batch_size 20, {prec}")
    cfg = tiny_cfg(fmd, layers=2, vocab=1024)
    w = fmd.synthetic_weights(cfg, seed=51)
    gpu = fmd.Qwen3(cfg, prec, max_len=256).load(w)
    rng = np.random.default_rng(52)
    prompts = [rng.integers(0, cfg.vocab_size, int(n)).tolist() for n in rng.integers(5, 61, 25)]
    force = rng.integers(2, 12, 25).tolist()
    budget = 10
    eng = fmd.Engine(gpu, fmd.EngineConfig(max_new_tokens=budget, max_batch_size=20, eos_id=EOS))
    res, stats = eng.generate(prompts, force_eot_step=force)
    assert stats.micro_batches == 2
    assert all(r.error is None for r in res)
    order = sorted(range(25), key=lambda i: len(prompts[i]))
    ref = orc.OracleModel(cfg, OPREC[prec], 256).load(w)
    for members in (order[:20], order[20:]):
        sub = [prompts[i] for i in members]
        n = check_greedy([(res[i].tokens, int(res[i].finish_reason)) for i in members], ref, sub,
                         budget, EOS, TOL[prec], force=[force[i] for i in members])
        assert n >= len(members)
        # the same micro-batch through generate_batch (20 rows at once)
        alone = gpu.generate_batch(sub, budget, eos=EOS, force_eot_step=[force[i] for i in members])
        assert [g.tokens for g in alone] == [res[i].tokens for i in members]


def test_failed_micro_batch_reports_the_library_message(fmd):
    _announce("engine error text and the RoPE table bound")
    cfg = tiny_cfg(fmd, layers=1, vocab=1024)
    w = fmd.synthetic_weights(cfg, seed=53)
    gpu = fmd.Qwen3(cfg, "int8", max_len=64).load(w)
    rng = np.random.default_rng(54)
    short = [rng.integers(0, 1000, 10).tolist() for _ in range(3)]
    long = [rng.integers(0, 1000, 40).tolist() for _ in range(2)]
    eng = fmd.Engine(gpu, fmd.EngineConfig(max_new_tokens=40, max_batch_size=3, eos_id=EOS))
    # micro-batch 1 (3 x 10 tokens) fits the table: 10 + 39 positions < 64;
    # micro-batch 2 (2 x 40 tokens) would write position 64 at its 25th
    # decode step while its rows are still generating
    res, stats = eng.generate(short + long)
    assert stats.micro_batches == 2
    assert all(r.error is None for r in res[:3])
    for r in res[3:]:
        assert r.error is not None and r.error.startswith("batch generation failed: "), r.error
        assert "rope position 64" in r.error, r.error
        assert r.tokens == []
    # with every row stopping before the table ends, the same batch succeeds
    res, _ = eng.generate(long, force_eot_step=[3, 20])
    assert all(r.error is None for r in res)
    assert [len(r.tokens) <= f for r, f in zip(res, [3, 20])] == [True, True]
    # generate_batch raises with the same message
    with pytest.raises(fmd.FmdError, match="rope position 64"):
        gpu.generate_batch(long, 40, eos=EOS)


def test_decode_entry_points_reject_pads_outside_the_cache(fmd):
    _announce("pad checks of decode_step / decode_loop / prefill")
    cfg = tiny_cfg(fmd, layers=1, vocab=1024)
    w = fmd.synthetic_weights(cfg, seed=55)
    gpu = fmd.Qwen3(cfg, "bf16", max_len=128).load(w)
    kv = gpu.new_caches(2, 64)
    kv.fill_random(3, 10)
    for pad in ([-1, 0], [0, 11]):
        with pytest.raises(fmd.FmdError, match="pad outside the cache") as e:
            gpu.decode_step([1, 2], kv, pad)
        assert e.value.code == -1
        with pytest.raises(fmd.FmdError, match="pad outside the cache"):
            gpu.decode_loop(kv, [1, 2], pad, 3, eos=EOS)
    assert kv.len() == 10
    # the cache is untouched by the rejected calls: a valid step still works
    logits = gpu.decode_step([1, 2], kv, [0, 10])
    assert np.all(np.isfinite(logits)) and kv.len() == 11
    # a prefill block that is padding in every row has no prompt
    kv2 = gpu.new_caches(2, 64)
    emb = np.zeros((2, 8, cfg.hidden_size), dtype=np.uint16)
    with pytest.raises(fmd.FmdError, match="empty prompt"):
        gpu.prefill(emb, kv2, [8, 8])
    assert kv2.len() == 0


@pytest.mark.parametrize("prec", ["int8", "bf16"])
def test_generate_after_finished_steps_is_unchanged(fmd, prec):
    """A greedy loop keeps up to two steps in flight, so it usually runs a
    step or two after every row is done.  Those launches must not leave
    exchange words that a later call could take for its own: the same
    generation run again (and after other generations) gives the same
    tokens."""
    _announce(f"generation after all-done steps, {prec}")
    cfg = tiny_cfg(fmd, layers=2, vocab=1024)
    w = fmd.synthetic_weights(cfg, seed=56)
    gpu = fmd.Qwen3(cfg, prec, max_len=512).load(w)
    rng = np.random.default_rng(57)
    prompts = [rng.integers(0, cfg.vocab_size, int(n)).tolist() for n in (40, 13, 77, 60)]
    first = gpu.generate_batch(prompts, 30, eos=EOS, force_eot_step=[3, 2, 4, 3])
    for _ in range(3):
        other = [rng.integers(0, cfg.vocab_size, 50).tolist() for _ in range(4)]
        gpu.generate_batch(other, 12, eos=EOS, force_eot_step=[1, 1, 1, 1])
        again = gpu.generate_batch(prompts, 30, eos=EOS, force_eot_step=[3, 2, 4, 3])
        assert [g.tokens for g in again] == [g.tokens for g in first]
