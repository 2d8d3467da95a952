"""A second, independent CPU restatement of the reference decoder in torch,
built from library routines: F.rms_norm, BLAS matmul, softmax over an
explicitly expanded (repeat_kv) head layout, torch's cos/sin.  Used only to
pin the C oracle on small configurations (qwen3.rs:111-145, 203-340,
444-511, 523-562; engine.rs:463-559).

`act` selects the activation dtype: every op computes in fp32 and its output
is rounded to that dtype, as the reference's tensors are (qwen3.rs:213-339):
the projections, norms, RoPE, the scores and the scaled scores, the softmax
probabilities, the context, silu, the gated product and the residual sums.
With a bf16/f16 `act` it differs from the oracle only in the fp32 summation
order of BLAS, so their distance is the floor any two implementations of the
same rounding model reach.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

P = "model.language_model."


def _w(weights, name):
    return weights[P + name]


class TorchQwen3:
    def __init__(self, cfg, weights, max_len=512, act=torch.float32, exact=()):
        """`exact`: names of weights kept as given (e.g. dequantised Q8_0
        rows, which the activation dtype need not represent)."""
        self.cfg = cfg
        self.act = act
        self.w = {}
        for k, v in weights.items():
            t = torch.from_numpy(np.asarray(v, dtype=np.float32))
            self.w[k] = t if k in exact else t.to(act).float()
        self.head = self.w.get(P + "lm_head.weight", self.w[P + "embed_tokens.weight"])
        hd = cfg.head_dim
        inv = torch.tensor(
            [1.0 / math.pow(cfg.rope_theta, 2.0 * i / hd) for i in range(hd // 2)],
            dtype=torch.float64).to(torch.float32)
        pos = torch.arange(max_len, dtype=torch.float32)[:, None]
        freqs = pos * inv[None, :]
        self.cos, self.sin = self.rd(freqs.cos()), self.rd(freqs.sin())

    def rd(self, x):
        return x if self.act == torch.float32 else x.to(self.act).float()

    def rope(self, x, positions):
        # x (b, h, t, hd); rotate-half with halves [0, hd/2), [hd/2, hd)
        c = self.cos[positions][None, None]
        s = self.sin[positions][None, None]
        half = x.shape[-1] // 2
        x1, x2 = x[..., :half], x[..., half:]
        return self.rd(torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1))

    def layer(self, i, x, kcache, vcache, offset, pad):
        cfg = self.cfg
        b, t, H = x.shape
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        p = f"layers.{i}."
        rd = self.rd
        h = rd(F.rms_norm(x, (H,), _w(self.w, p + "input_layernorm.weight"), eps))
        q = rd(h @ _w(self.w, p + "self_attn.q_proj.weight").T)
        k = rd(h @ _w(self.w, p + "self_attn.k_proj.weight").T)
        v = rd(h @ _w(self.w, p + "self_attn.v_proj.weight").T)
        q = rd(F.rms_norm(q.view(b, t, nh, hd), (hd,), _w(self.w, p + "self_attn.q_norm.weight"), eps))
        k = rd(F.rms_norm(k.view(b, t, nkv, hd), (hd,), _w(self.w, p + "self_attn.k_norm.weight"), eps))
        v = v.view(b, t, nkv, hd)
        positions = torch.arange(offset, offset + t)
        q = self.rope(q.transpose(1, 2), positions)
        k = self.rope(k.transpose(1, 2), positions)
        kcache[i][:, :, offset:offset + t] = k
        vcache[i][:, :, offset:offset + t] = v.transpose(1, 2)
        L = offset + t
        kk = kcache[i][:, :, :L].repeat_interleave(nh // nkv, dim=1)
        vv = vcache[i][:, :, :L].repeat_interleave(nh // nkv, dim=1)
        scores = rd(rd(q @ kk.transpose(-1, -2)) * rd(torch.tensor(1.0 / math.sqrt(hd))))
        allowed = torch.zeros(b, 1, t, L, dtype=torch.bool)
        for bi in range(b):
            for qi in range(t):
                aq = offset + qi
                lo = pad[bi] if aq >= pad[bi] else 0
                allowed[bi, 0, qi, lo:aq + 1] = True
        scores = scores.masked_fill(~allowed, float("-inf"))
        ctx = rd(rd(torch.softmax(scores, dim=-1)) @ vv)
        ctx = ctx.transpose(1, 2).reshape(b, t, nh * hd)
        x = rd(x + rd(ctx @ _w(self.w, p + "self_attn.o_proj.weight").T))
        h = rd(F.rms_norm(x, (H,), _w(self.w, p + "post_attention_layernorm.weight"), eps))
        g = rd(h @ _w(self.w, p + "mlp.gate_proj.weight").T)
        u = rd(h @ _w(self.w, p + "mlp.up_proj.weight").T)
        a = rd(rd(F.silu(g)) * u)
        return rd(x + rd(a @ _w(self.w, p + "mlp.down_proj.weight").T))

    def forward(self, x, kc, vc, offset, pad):
        for i in range(self.cfg.num_hidden_layers):
            x = self.layer(i, x, kc, vc, offset, pad)
        x = self.rd(F.rms_norm(x, (self.cfg.hidden_size,), _w(self.w, "norm.weight"),
                               self.cfg.rms_norm_eps))
        return self.rd(x[:, -1] @ self.head.T)

    def generate(self, prompts, budget, eos, force=None):
        cfg = self.cfg
        E = _w(self.w, "embed_tokens.weight")
        b = len(prompts)
        total = max(len(p) for p in prompts)
        pad = [total - len(p) for p in prompts]
        x = torch.zeros(b, total, cfg.hidden_size)
        for i, p in enumerate(prompts):
            if len(p):
                x[i, pad[i]:] = E[torch.tensor(p, dtype=torch.long)]
        cap = total + budget
        kc = [torch.zeros(b, cfg.num_key_value_heads, cap, cfg.head_dim) for _ in range(cfg.num_hidden_layers)]
        vc = [torch.zeros_like(t) for t in kc]
        logits = self.forward(x, kc, vc, 0, pad)
        off = total
        out = [[] for _ in range(b)]
        fin = [0] * b
        done = [False] * b
        all_logits = [logits]
        for step in range(budget):
            nxt = logits.argmax(-1).tolist()
            all_done = True
            for i in range(b):
                if done[i]:
                    continue
                tok = nxt[i]
                if force is not None and force[i] == step:
                    tok = eos
                if tok == eos:
                    done[i] = True
                    fin[i] = 1
                else:
                    out[i].append(tok)
                    all_done = False
            if all_done or step + 1 == budget:
                break
            feed = [eos if done[i] else nxt[i] for i in range(b)]
            logits = self.forward(E[torch.tensor(feed)][:, None], kc, vc, off, pad)
            all_logits.append(logits)
            off += 1
        return out, fin, all_logits
