"""A second, independent CPU restatement of the reference's audio path in
torch, built from library routines: F.conv1d, F.gelu (exact erf form),
F.layer_norm, F.silu, torch.softmax and BLAS matmul.  Used only to pin the C
oracle (whisper_encoder.rs:44-163, adaptor.rs:41-64, mod.rs:82-126).

`act` selects the activation dtype: every op computes in fp32 and its output
is rounded to that dtype, at the points where the reference's tensors are:
the mel cast, each conv and its bias and gelu, the positions sum, the norms,
each projection and its bias, the q/k scaling by head_dim^-1/4 (the
multiplier itself rounded to the dtype), the scores, the probabilities, the
context, the residual sums, silu and the adaptor's layers.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

E = "model.whisper_encoder."
A = "model.vq_adaptor."


class TorchWhisper:
    def __init__(self, cfg, weights, act=torch.float32):
        self.cfg = cfg
        self.act = act
        self.w = {k: self.rd(torch.from_numpy(np.asarray(v, dtype=np.float32)))
                  for k, v in weights.items()}

    def rd(self, x):
        return x if self.act == torch.float32 else x.to(self.act).float()

    def lin(self, x, name, bias=True):
        y = self.rd(x @ self.w[name + ".weight"].T)
        return self.rd(y + self.w[name + ".bias"]) if bias else y

    def ln(self, x, name, eps):
        return self.rd(F.layer_norm(x, (x.shape[-1],), self.w[name + ".weight"],
                                    self.w[name + ".bias"], eps))

    def stem(self, mel):
        rd = self.rd
        x = rd(torch.from_numpy(np.asarray(mel, dtype=np.float32)))
        h = rd(F.conv1d(x, self.w[E + "conv1.weight"], padding=1))
        h = rd(F.gelu(rd(h + self.w[E + "conv1.bias"][None, :, None]), approximate="none"))
        h = rd(F.conv1d(h, self.w[E + "conv2.weight"], padding=1, stride=2))
        h = rd(F.gelu(rd(h + self.w[E + "conv2.bias"][None, :, None]), approximate="none"))
        h = h.transpose(1, 2)
        t = h.shape[1]
        return rd(h + self.w[E + "embed_positions.weight"][:t][None])

    def layer(self, i, x):
        cfg, rd = self.cfg, self.rd
        p = E + f"layers.{i}."
        b, t, d = x.shape
        nh = cfg.encoder_attention_heads
        hd = d // nh
        s = self.rd(torch.tensor(float(hd) ** -0.25, dtype=torch.float32))
        h = self.ln(x, p + "self_attn_layer_norm", 1e-5)
        q = rd(self.lin(h, p + "self_attn.q_proj") * s)
        k = rd(self.lin(h, p + "self_attn.k_proj", bias=False) * s)
        v = self.lin(h, p + "self_attn.v_proj")
        q = q.view(b, t, nh, hd).transpose(1, 2)
        k = k.view(b, t, nh, hd).transpose(1, 2)
        v = v.view(b, t, nh, hd).transpose(1, 2)
        scores = rd(q @ k.transpose(-1, -2))
        probs = rd(torch.softmax(scores, dim=-1))
        ctx = rd(probs @ v).transpose(1, 2).reshape(b, t, d)
        x = rd(x + self.lin(ctx, p + "self_attn.out_proj"))
        h = self.ln(x, p + "final_layer_norm", 1e-5)
        f = rd(F.gelu(self.lin(h, p + "fc1"), approximate="none"))
        return rd(x + self.lin(f, p + "fc2"))

    def forward(self, mel, layers=None):
        x = self.stem(mel)
        n = self.cfg.encoder_layers if layers is None else layers
        for i in range(n):
            x = self.layer(i, x)
        return self.ln(x, E + "layer_norm", 1e-5)

    def adaptor(self, frames):
        m = self.cfg.audio_merge_size
        f = torch.as_tensor(np.asarray(frames, dtype=np.float32))
        g = f.shape[0] // m
        merged = f[: g * m].reshape(g, m * f.shape[1])
        h = self.rd(F.silu(self.lin(merged, A + "layers.0")))
        h = self.lin(h, A + "layers.2")
        return self.ln(h, A + "layers.3", self.cfg.norm_eps)
