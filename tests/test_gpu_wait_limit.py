"""The bounded waits of the single-launch decode attention.

With a spin limit of 0 (fmd_dec_set_spin_limit), a wait that is not met at
its first poll gives up at once.  The launch must still drain, the call must
fail with the spin-limit error instead of hanging, and the steps before the
first failure must match a run with the default limit.  Restoring the limit
makes the next steps succeed again (the epoch advanced through the failed
launch, so no stale exchange word is taken for a fresh one).
"""
import numpy as np
import pytest

from tests.gpu_util import TOL, tiny_cfg

pytestmark = pytest.mark.gpu


def _steps(fmd, gpu, cfg, limit, steps=6):
    rng = np.random.default_rng(8)
    lens = [200, 37, 120, 300]
    P = max(lens)
    kv = gpu.new_caches(len(lens), P + steps + 4)
    kv.fill_random(seed=9, length=P)
    pad = [P - n for n in lens]
    gpu.set_spin_limit(limit)
    logits, errors = {}, []
    for s in range(steps):
        ids = rng.integers(0, cfg.vocab_size, len(lens)).tolist()
        try:
            logits[s] = gpu.decode_step(ids, kv, pad)
        except fmd.FmdError as e:
            errors.append((s, str(e)))
            kv.set_len(P + s + 1)
    gpu.set_spin_limit(20000)
    return logits, errors, kv, pad


def test_wait_error_path_drains_and_reports(fmd):
    print("[gpu] spin limit 0 on the tiny int8 decoder", flush=True)
    cfg = tiny_cfg(fmd)
    gpu = fmd.Qwen3(cfg, "int8", max_len=1024).load(fmd.synthetic_weights(cfg, seed=7))
    base, base_err, _, _ = _steps(fmd, gpu, cfg, 20000)
    assert not base_err and len(base) == 6
    got, errors, kv, pad = _steps(fmd, gpu, cfg, 0)
    for _, e in errors:
        assert "did not meet within the spin limit" in e, e
    # a failed step still appends its (possibly wrong) K/V, so only the steps
    # before the first failure must reproduce the normal run
    first_err = errors[0][0] if errors else 6
    for s, lg in got.items():
        if s < first_err:
            d = np.max(np.abs(lg - base[s]))
            assert d < TOL["int8"], (s, d)
    # the default limit works again on the same handle
    after = gpu.decode_step([1, 2, 3, 4], kv, pad)
    assert np.all(np.isfinite(after))
    with pytest.raises(fmd.FmdError):
        gpu.set_spin_limit(-1)
    if not errors:
        pytest.skip("every wait was satisfied at its first poll")
