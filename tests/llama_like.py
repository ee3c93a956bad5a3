"""A seeded Llama/Qwen-shaped torch decoder used only as test scaffolding: it has the
module layout the reference's paged forward loop walks (model.model.embed_tokens,
.layers[i].{input_layernorm, self_attn.{q_proj, k_proj, v_proj, o_proj, q_norm, k_norm,
rope, num_heads, num_kv_heads, head_dim, window, scale}, mlp, post_attention_layernorm},
model.model.norm, model.lm_head, model.config). Not part of the product."""

from types import SimpleNamespace

import torch
from torch import nn


class RMSNorm(nn.Module):
    def __init__(self, width, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(width))
        self.eps = eps

    def forward(self, x):
        y = x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class RotaryEmbedding(nn.Module):
    """Rotate-half RoPE on ``[B, H, T, D]`` at absolute ``positions [B, T]``."""

    def __init__(self, head_dim, base=10000.0):
        super().__init__()
        self.register_buffer("inv_freq", 1.0 / base ** (torch.arange(0, head_dim, 2).float()
                                                         / head_dim), persistent=False)

    def forward(self, x, positions):
        angle = positions[:, None, :, None].float() * self.inv_freq
        cos, sin = angle.cos(), angle.sin()
        half = x.shape[-1] // 2
        a, b = x[..., :half].float(), x[..., half:].float()
        return torch.cat([a * cos - b * sin, a * sin + b * cos], -1).to(x.dtype)


class Attention(nn.Module):
    def __init__(self, hidden, heads, kv_heads, head_dim, window, qk_norm):
        super().__init__()
        self.num_heads, self.num_kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.window, self.scale = window, head_dim ** -0.5
        self.q_proj = nn.Linear(hidden, heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden, kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden, kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(heads * head_dim, hidden, bias=False)
        self.q_norm = RMSNorm(head_dim) if qk_norm else nn.Identity()
        self.k_norm = RMSNorm(head_dim) if qk_norm else nn.Identity()
        self.rope = RotaryEmbedding(head_dim)


class MLP(nn.Module):
    def __init__(self, hidden, ffn):
        super().__init__()
        self.gate_proj = nn.Linear(hidden, ffn, bias=False)
        self.up_proj = nn.Linear(hidden, ffn, bias=False)
        self.down_proj = nn.Linear(ffn, hidden, bias=False)

    def forward(self, x):
        return self.down_proj(nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, hidden, heads, kv_heads, head_dim, ffn, window, qk_norm):
        super().__init__()
        self.input_layernorm = RMSNorm(hidden)
        self.self_attn = Attention(hidden, heads, kv_heads, head_dim, window, qk_norm)
        self.post_attention_layernorm = RMSNorm(hidden)
        self.mlp = MLP(hidden, ffn)


class Body(nn.Module):
    def __init__(self, vocab, hidden, layers):
        super().__init__()
        self.embed_tokens = nn.Embedding(vocab, hidden)
        self.layers = nn.ModuleList(layers)
        self.norm = RMSNorm(hidden)


class LlamaLike(nn.Module):
    """``windows``: per-layer sliding window (None = full attention); ``qk_norm``: Qwen3's
    per-head RMSNorm on q and k."""

    def __init__(self, *, vocab=97, hidden=256, heads=8, kv_heads=2, head_dim=64, ffn=512,
                 windows=(None, 24), qk_norm=True, seed=0, max_positions=4096):
        super().__init__()
        torch.manual_seed(seed)
        layers = [DecoderLayer(hidden, heads, kv_heads, head_dim, ffn, w, qk_norm)
                  for w in windows]
        self.model = Body(vocab, hidden, layers)
        self.lm_head = nn.Linear(hidden, vocab, bias=False)
        self.config = SimpleNamespace(vocab_size=vocab, max_position_embeddings=max_positions,
                                      attention_dropout=0.0)
        with torch.no_grad():
            for p in self.parameters():
                if p.ndim == 2:
                    p.normal_(0.0, p.shape[-1] ** -0.5)
            for m in self.modules():
                if isinstance(m, RMSNorm):
                    m.weight.uniform_(0.8, 1.2)
