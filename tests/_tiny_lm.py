"""A seeded, randomly initialised decoder-only LM with the mlx-lm model
conventions the decode closure relies on (``model(tokens, cache=caches)``,
``cache.update_and_fetch``, ``cache.offset`` for RoPE, ``model.layers``,
attention through ``F.scaled_dot_product_attention``).  Test scaffolding
only: no checkpoint, fp32 weights."""

import torch
import torch.nn as nn
import torch.nn.functional as F


def _rope(x, offset, base=10000.0):
    """Rotary embedding on (B, H, L, D), positions offset .. offset+L-1;
    ``offset`` is an int or a 0-d integer device tensor (graph-captured
    decode keeps it on the device)."""
    B, H, L, D = x.shape
    half = D // 2
    inv = base ** (-torch.arange(half, device=x.device, dtype=torch.float32) / half)
    pos = torch.arange(L, device=x.device, dtype=torch.float32) + offset
    ang = pos[:, None] * inv[None, :]
    cos, sin = ang.cos().to(x.dtype), ang.sin().to(x.dtype)
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


class Attention(nn.Module):
    def __init__(self, dim, n_heads, n_kv_heads, head_dim, qk_gain):
        super().__init__()
        self.h, self.hkv, self.d = n_heads, n_kv_heads, head_dim
        self.q_proj = nn.Linear(dim, n_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(dim, n_kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(dim, n_kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(n_heads * head_dim, dim, bias=False)
        with torch.no_grad():
            self.q_proj.weight.mul_(qk_gain)
            self.k_proj.weight.mul_(qk_gain)

    def forward(self, x, cache):
        B, L, _ = x.shape
        q = self.q_proj(x).view(B, L, self.h, self.d).transpose(1, 2)
        k = self.k_proj(x).view(B, L, self.hkv, self.d).transpose(1, 2)
        v = self.v_proj(x).view(B, L, self.hkv, self.d).transpose(1, 2)
        off = cache.offset
        q, k = _rope(q, off), _rope(k, off)
        k, v = cache.update_and_fetch(k.contiguous(), v.contiguous())
        g = self.h // self.hkv
        k = k.repeat_interleave(g, dim=1).contiguous()
        v = v.repeat_interleave(g, dim=1).contiguous()
        o = F.scaled_dot_product_attention(q.contiguous(), k, v, is_causal=L > 1, scale=self.d ** -0.5)
        return self.o_proj(o.transpose(1, 2).reshape(B, L, self.h * self.d))


class Block(nn.Module):
    def __init__(self, dim, n_heads, n_kv_heads, head_dim, qk_gain):
        super().__init__()
        self.n1 = nn.LayerNorm(dim)
        self.attn = Attention(dim, n_heads, n_kv_heads, head_dim, qk_gain)
        self.n2 = nn.LayerNorm(dim)
        self.mlp = nn.Sequential(nn.Linear(dim, 2 * dim), nn.GELU(), nn.Linear(2 * dim, dim))

    def forward(self, x, cache):
        x = x + self.attn(self.n1(x), cache)
        return x + self.mlp(self.n2(x))


class TinyLM(nn.Module):
    def __init__(self, vocab=97, dim=128, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64,
                 qk_gain=1.0, seed=0):
        super().__init__()
        g = torch.random.fork_rng(devices=[])
        with g:
            torch.manual_seed(seed)
            self.embed = nn.Embedding(vocab, dim)
            self.layers = nn.ModuleList(Block(dim, n_heads, n_kv_heads, head_dim, qk_gain)
                                        for _ in range(n_layers))
            self.norm = nn.LayerNorm(dim)
            self.head = nn.Linear(dim, vocab, bias=False)

    def forward(self, tokens, cache):
        x = self.embed(tokens)
        for blk, c in zip(self.layers, cache):
            x = blk(x, c)
        return self.head(self.norm(x))


class ByteTokenizer:
    """encode: bytes mod vocab; decode: space-joined ids.  No EOS."""

    eos_token_id = None

    def __init__(self, vocab=97):
        self.vocab = vocab

    def encode(self, text):
        return [b % self.vocab for b in text.encode()]

    def decode(self, ids):
        return " ".join(str(i) for i in ids)
