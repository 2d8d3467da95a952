"""Child process of the GPU tests that need their own environment (the
decoder reads its tuning and test knobs once per process).

Usage: gpu_child.py CFG PREC STEPS OUT.npz [prefill]
Runs STEPS decode steps over a randomly filled cache with seeded token ids
(the same ids whatever the outputs, so runs under different knobs see the
same inputs), saves the logits of the steps that succeeded to OUT.npz and
prints one JSON line with the step errors.  With `prefill`, it instead
prefills seeded ragged prompts (chunk 512, so the packed chunks hold
hundreds of rows) and saves the logits and every layer's K and V."""
from __future__ import annotations

import importlib
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def main() -> None:
    import numpy as np

    from tests.gpu_util import small_cfg, tiny_cfg

    cfg_name, prec, steps, out_path = sys.argv[1], sys.argv[2], int(sys.argv[3]), sys.argv[4]
    fmd = importlib.import_module("fast-moss-diarization_amd")
    cfg = tiny_cfg(fmd) if cfg_name == "tiny" else small_cfg(fmd)
    gpu = fmd.Qwen3(cfg, prec, max_len=1024).load(fmd.synthetic_weights(cfg, seed=7))
    if len(sys.argv) > 5 and sys.argv[5] == "prefill":
        rng = np.random.default_rng(10)
        lens = [1000, 41, 900, 700, 1, 650, 800, 520]  # 1654 rows in the first chunk
        T = max(lens)
        emb = np.zeros((len(lens), T, cfg.hidden_size), dtype=gpu.precision.numpy_storage)
        for b, n in enumerate(lens):
            emb[b, T - n:] = gpu.embed(rng.integers(0, cfg.vocab_size, n))
        kv = gpu.new_caches(len(lens), T + 4)
        logits = gpu.prefill(emb, kv, [T - n for n in lens], chunk=512)
        cache = np.stack([np.stack([kv.read(layer, which) for which in (0, 1)])
                          for layer in range(cfg.num_hidden_layers)])
        np.savez(out_path, logits=logits, steps=np.zeros(0, np.int32), cache=cache)
        print(json.dumps({"errors": [], "len": kv.len()}), flush=True)
        return
    rng = np.random.default_rng(8)
    lens = [200, 37, 120, 300]
    P = max(lens)
    kv = gpu.new_caches(len(lens), P + steps + 4)
    kv.fill_random(seed=9, length=P)
    pad = [P - n for n in lens]
    logits, ok, errors = [], [], []
    for s in range(steps):
        ids = rng.integers(0, cfg.vocab_size, len(lens)).tolist()
        try:
            logits.append(gpu.decode_step(ids, kv, pad))
            ok.append(s)
        except fmd.FmdError as e:
            errors.append(str(e))
            kv.set_len(P + s + 1)
    np.savez(out_path, logits=np.asarray(logits, dtype=np.float32).reshape(len(ok), len(lens), cfg.vocab_size),
             steps=np.asarray(ok, dtype=np.int32))
    print(json.dumps({"errors": errors, "len": kv.len()}), flush=True)


if __name__ == "__main__":
    main()
