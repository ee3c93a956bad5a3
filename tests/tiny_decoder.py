"""A seeded toy GQA decoder (RMSNorm, RoPE, SiLU MLP) used only as test scaffolding
for the runner integration: it produces realistic per-layer q/k/v for a paged
forward step. Not part of the product."""

import math

import torch


class TinyDecoder:
    def __init__(self, device, *, vocab=101, layers=2, hq=4, hkv=2, d=64, ffn=384, seed=0):
        g = torch.Generator().manual_seed(seed)
        h = hq * d
        self.vocab, self.layers, self.hq, self.hkv, self.d, self.h = vocab, layers, hq, hkv, d, h
        self.scale = d ** -0.5

        def w(*shape):
            return (torch.randn(*shape, generator=g) / math.sqrt(shape[0])).to(device)

        self.embed = torch.randn(vocab, h, generator=g).to(device)
        self.blocks = [dict(wq=w(h, hq * d), wk=w(h, hkv * d), wv=w(h, hkv * d), wo=w(hq * d, h),
                            w1=w(h, ffn), w3=w(h, ffn), w2=w(ffn, h)) for _ in range(layers)]
        self.head = w(h, vocab)
        inv = 1.0 / (10000 ** (torch.arange(0, d, 2).float() / d))
        self.inv_freq = inv.to(device)

    @staticmethod
    def rms(x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)

    def rope(self, x, pos):
        """x [T, H, d], pos [T] absolute positions (rotate-half RoPE)."""
        ang = pos[:, None].float() * self.inv_freq[None]
        cos, sin = ang.cos()[:, None], ang.sin()[:, None]
        a, b = x[..., : self.d // 2], x[..., self.d // 2:]
        return torch.cat([a * cos - b * sin, a * sin + b * cos], -1)

    def forward(self, ids, positions, attend):
        """ids/positions: packed [T] (rows in batch order); attend(layer, q, k, v) ->
        [T, hq, d]. Returns logits [T, vocab]."""
        x = self.embed[ids]
        T = x.shape[0]
        for i, p in enumerate(self.blocks):
            n = self.rms(x)
            q = self.rope((n @ p["wq"]).view(T, self.hq, self.d), positions)
            k = self.rope((n @ p["wk"]).view(T, self.hkv, self.d), positions)
            v = (n @ p["wv"]).view(T, self.hkv, self.d)
            o = attend(i, q.contiguous(), k.contiguous(), v.contiguous())
            x = x + o.reshape(T, -1).float() @ p["wo"]
            n2 = self.rms(x)
            x = x + (torch.nn.functional.silu(n2 @ p["w1"]) * (n2 @ p["w3"])) @ p["w2"]
        return self.rms(x) @ self.head
