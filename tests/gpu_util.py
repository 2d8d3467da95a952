"""Shared helpers of the GPU parity tests: build the HIP decoder and the CPU
oracle from one synthetic checkpoint and compare their outputs."""
from __future__ import annotations

import numpy as np
import torch

TOL = {"f32": 1e-4, "f16": 2e-2, "bf16": 2e-2, "int8": 2e-2}
OPREC = {"f32": 0, "f16": 1, "bf16": 2, "int8": 3}
P = "model.language_model."


def tiny_cfg(fmd, layers=2, vocab=1024):
    return fmd.TextConfig(vocab_size=vocab, hidden_size=256, intermediate_size=512,
                          num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                          head_dim=128, rope_theta=1e6)


def small_cfg(fmd, layers=2, vocab=2048):
    """Full Qwen3-0.6B layer widths, fewer layers and a smaller vocabulary."""
    return fmd.TextConfig(vocab_size=vocab, hidden_size=1024, intermediate_size=3072,
                          num_hidden_layers=layers, num_attention_heads=16, num_key_value_heads=8,
                          head_dim=128, rope_theta=1e6)


def build_pair(fmd, orc, cfg, prec: str, seed=0, max_len=8192, weights=None):
    w = weights if weights is not None else fmd.synthetic_weights(cfg, seed=seed)
    gpu = fmd.Qwen3(cfg, prec, max_len=max_len).load(w)
    ref = orc.OracleModel(cfg, OPREC[prec], max_len).load(w)
    return gpu, ref, w


def storage_to_f32(a: np.ndarray, prec: str) -> np.ndarray:
    if prec == "bf16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def f32_to_storage(x: np.ndarray, prec: str, orc) -> np.ndarray:
    return orc.to_storage(x, OPREC[prec])


def top2_margin(logits: np.ndarray) -> np.ndarray:
    s = np.sort(logits, axis=-1)
    return s[..., -1] - s[..., -2]


def check_greedy(gpu_out, ref_model, prompts, budget, eos, tol, force=None, block=256):
    """Tokens must agree wherever the oracle's top-2 logit margin exceeds tol.

    Replays the oracle along the GPU's own tokens; at the first step where a
    row differs, the oracle's margin there must be <= tol (a near-tie), after
    which that row is not compared further.  Returns the number of compared
    tokens."""
    emb, pad = ref_model.padded_embeds(prompts)
    b = len(prompts)
    kv = ref_model.new_kv(b, emb.shape[1] + budget)
    logits = ref_model.prefill(kv, emb, pad, block=block)
    done = [False] * b
    diverged = [False] * b
    pos = [0] * b
    compared = 0
    for step in range(budget):
        ref_next = logits.argmax(-1)
        margins = top2_margin(logits)
        feed = []
        for i in range(b):
            toks, fin = gpu_out[i]
            if done[i] or diverged[i]:
                feed.append(eos)
                continue
            forced = force is not None and force[i] == step
            want = eos if forced else int(ref_next[i])
            have = toks[pos[i]] if pos[i] < len(toks) else eos
            if have != want:
                assert margins[i] <= tol, (
                    f"row {i} step {step}: device {have} vs oracle {want}, margin {margins[i]:.4g}")
                diverged[i] = True
                feed.append(eos)
                continue
            compared += 1
            if want == eos:
                done[i] = True
                assert fin == 1, f"row {i} should finish with Stop"
                feed.append(eos)
            else:
                pos[i] += 1
                feed.append(want)
        if all(d or v for d, v in zip(done, diverged)) or step + 1 == budget:
            break
        logits = ref_model.decode_step(kv, feed, pad)
    for i in range(b):
        if not diverged[i] and not done[i]:
            assert len(gpu_out[i][0]) == pos[i], f"row {i}: extra tokens"
    return compared


# --------------------------------------------------------------------------
# The fp32 summation-order floor
#
# The device, the C oracle and the reference all round every op's output to
# the activation dtype but sum their fp32 dot products in different orders.
# A rounding boundary turns a sub-ulp difference into a whole-ulp one, and the
# next layers carry it on, so over several 16-bit layers two correct
# implementations drift apart by a few activation ulps of the logits.  The
# torch twin (tests/torch_ref.py) implements the same rounding model with BLAS
# summation; its distance to the oracle on the same inputs measures that
# floor.  A logit gap above the bar passes only if it sits at the floor.


def torch_twin(orc, cfg, w, prec: str, max_len: int):
    from tests.torch_ref import TorchQwen3

    act = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16,
           "int8": torch.float16}[prec]
    exact = ()
    if prec == "int8":
        w = dict(w)
        for name, W in list(w.items()):
            if W.ndim == 2 and "embed_tokens" not in name:
                w[name] = orc.dequantize_q8_0(orc.quantize_q8_0(W), *W.shape)
        E = w[P + "embed_tokens.weight"]
        if P + "lm_head.weight" not in w:
            w[P + "lm_head.weight"] = orc.dequantize_q8_0(orc.quantize_q8_0(E), *E.shape)
        exact = tuple(n for n, W in w.items() if W.ndim == 2 and "embed_tokens" not in n)
    return TorchQwen3(cfg, w, max_len=max_len, act=act, exact=exact)


def snapshot_kv(ref_kv, layers: int):
    """The oracle cache's contents as torch tensors (for the twin)."""
    k = [torch.from_numpy(ref_kv.read(i, 0).copy()) for i in range(layers)]
    v = [torch.from_numpy(ref_kv.read(i, 1).copy()) for i in range(layers)]
    return k, v


def twin_decode_step(twin, kv_snapshot, ids, pad, offset):
    k, v = kv_snapshot
    E = twin.w[P + "embed_tokens.weight"]
    return twin.forward(E[torch.tensor(list(ids))][:, None], k, v, offset,
                        [int(x) for x in pad]).numpy()


def gap_stats(a: np.ndarray, b: np.ndarray) -> dict:
    d = np.abs(a.astype(np.float64) - b.astype(np.float64))
    return {"max": float(d.max()), "rms": float(np.sqrt(np.mean(d * d))),
            "p999": float(np.quantile(d, 0.999)), "frac": float(np.mean(d > 0))}


def assert_logits_match(got, want, prec: str, twin=None, what=""):
    """max |got - want| < TOL[prec]; above it, only at the measured floor:
    rms within 1.25x and max within 1.5x of |twin - want|."""
    g = gap_stats(got, want)
    line = f"[gap] {what} {prec}: device-oracle max {g['max']:.4g} rms {g['rms']:.3g}"
    if twin is not None:
        f = gap_stats(twin, want)
        line += f" | twin-oracle max {f['max']:.4g} rms {f['rms']:.3g}"
    print(line, flush=True)
    if g["max"] < TOL[prec]:
        return
    assert twin is not None, line
    assert g["rms"] <= 1.25 * f["rms"] and g["max"] <= 1.5 * f["max"], line


def assert_greedy_match(got, want, prec: str, twin=None):
    """Greedy ids (argmax, first index on ties) agree wherever the oracle's
    top-2 margin exceeds the bar TOL[prec].  With a twin (a second correct
    implementation of the same rounding model, tests/torch_ref.py), a device
    flip above the bar is accepted only on evidence that two correct
    implementations disagree there: the twin flips the same row too, or that
    row's margin is below the row's own twin-oracle distance max |twin -
    oracle| (a gap that large can reorder the top two).  The device's and the
    twin's flips are printed side by side."""
    bar = TOL[prec]
    s = np.sort(want, axis=-1)
    margin = s[:, -1] - s[:, -2]
    ref_ids = want.argmax(-1)
    flips = [(b, float(margin[b])) for b in range(want.shape[0])
             if int(got[b].argmax()) != int(ref_ids[b])]
    line = f"[greedy] {prec}: bar {bar:.4g}, device flips {flips}"
    twin_flips, row_gap = set(), None
    if twin is not None:
        twin_flips = {b for b in range(want.shape[0]) if int(twin[b].argmax()) != int(ref_ids[b])}
        row_gap = np.max(np.abs(twin - want), axis=-1)
        line += (f", twin flips {[(b, float(margin[b])) for b in sorted(twin_flips)]}, "
                 f"row twin-oracle gaps {[round(float(g), 4) for g in row_gap]}")
    print(line, flush=True)
    for b, m in flips:
        if m <= bar:
            continue
        assert twin is not None, (b, m, bar)
        assert b in twin_flips or m <= float(row_gap[b]), (b, m, float(row_gap[b]))
