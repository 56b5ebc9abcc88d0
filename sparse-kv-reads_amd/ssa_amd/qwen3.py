"""A minimal Qwen3 decoder with the engine's decode-attention seam, random-init weights.

The reference drives its path from an external engine (``specd``'s ``Qwen3Model``, not under the
reference tree); its tests use that engine's model surface (tests/_tiny_model.py:20-62): a
``Qwen3Model`` with ``layers[i].attn`` modules carrying ``decode_attn_op``, ``embed``,
``final_norm``, ``lm_head`` (None when tied), ``rope_cos`` / ``rope_sin`` tables,
``alloc_cache(max_len)`` with ``k`` / ``v`` lists of ``[B, H_kv, L, d]`` tensors and
``cur_len``, and ``model(ids, cache, start_pos=0)`` returning logits. This module provides that
surface so the seam (``ssa_amd.patch``) and the graph decoder (``ssa_amd.graph_decode``) have a
model to run: embedding, RMSNorm, q/k/v/o projections with per-head q/k RMSNorm, rotary
embedding (half-split), SwiGLU MLP, tied LM head.

Projections and the MLP are library GEMMs (torch on hipBLASLt). Prompt attention is exact causal
attention computed in fp32 chunks; single-token decode calls ``decode_attn_op`` when one is
installed, else the dense split-K HIP kernel on a GPU (fp32 torch on the CPU).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn


@dataclass(frozen=True)
class Qwen3Config:
    vocab_size: int = 151936
    hidden_size: int = 1024
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    max_position_embeddings: int = 40960
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    tie_word_embeddings: bool = True


QWEN3_0_6B = Qwen3Config()
QWEN3_4B = Qwen3Config(hidden_size=2560, num_hidden_layers=36, num_attention_heads=32, num_key_value_heads=8,
                       intermediate_size=9728)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


def rope_tables(max_pos: int, d: int, theta: float, device=None):
    """cos, sin ``[max_pos, d/2]`` fp32 of the half-split rotary embedding."""
    inv = theta ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    return ang.cos().float().to(device), ang.sin().float().to(device)


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Rotate ``q [B, H, T, d]`` and ``k [B, H_kv, T, d]`` by the angles of their ``T`` positions
    (``cos``, ``sin [T, d/2]``): pairs (x_i, x_{i+d/2})."""
    def rot(x):
        xf = x.float()
        h = xf.shape[-1] // 2
        x1, x2 = xf[..., :h], xf[..., h:]
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1).to(x.dtype)
    return rot(q), rot(k)


def causal_attention(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, start: int, *, chunk: int = 1024):
    """Exact causal attention in fp32: query ``t`` of ``q [B, H, T, d]`` sits at position
    ``start + t`` and sees keys ``[0, start + t]`` of ``K, V [B, H_kv, n, d]``. Returns
    ``[B, H, T, d]`` in q's dtype."""
    B, H, T, d = q.shape
    Hk = K.shape[1]
    G = H // Hk
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(d)
    for b in range(B):
        for t0 in range(0, T, chunk):
            t1 = min(T, t0 + chunk)
            n1 = start + t1                                            # keys the chunk can see
            qf = q[b, :, t0:t1].float().reshape(Hk, G * (t1 - t0), d)
            kt = K[b, :, :n1].float().transpose(1, 2).contiguous()      # [Hk, d, n1]
            s = torch.matmul(qf, kt).view(Hk, G, t1 - t0, n1) * scale
            pos = torch.arange(start + t0, start + t1, device=q.device)
            s.masked_fill_(torch.arange(n1, device=q.device)[None, :] > pos[:, None], float("-inf"))
            p = torch.softmax(s, -1).view(Hk, G * (t1 - t0), n1)
            o = torch.matmul(p, V[b, :, :n1].float().contiguous())
            out[b, :, t0:t1] = o.view(H, t1 - t0, d).to(q.dtype)
    return out


class KVCache:
    """Per layer ``k[i], v[i] [B, H_kv, max_seq_len, d]``; positions ``[0, cur_len)`` are valid."""

    def __init__(self, cfg: Qwen3Config, max_len: int, batch: int, dtype, device):
        shape = (batch, cfg.num_key_value_heads, max_len, cfg.head_dim)
        self.k = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(cfg.num_hidden_layers)]
        self.v = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(cfg.num_hidden_layers)]
        self.cur_len = 0
        self.max_seq_len = max_len


class Attention(nn.Module):
    def __init__(self, cfg: Qwen3Config, layer_idx: int):
        super().__init__()
        H, Hk, d, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size
        self.H, self.H_kv, self.d, self.layer_idx = H, Hk, d, layer_idx
        self.q = nn.Linear(D, H * d, bias=False)
        self.k = nn.Linear(D, Hk * d, bias=False)
        self.v = nn.Linear(D, Hk * d, bias=False)
        self.o = nn.Linear(H * d, D, bias=False)
        self.q_norm = RMSNorm(d, cfg.rms_norm_eps)
        self.k_norm = RMSNorm(d, cfg.rms_norm_eps)
        self.decode_attn_op = None                 # the seam: set by ssa_amd.patch.install

    def forward(self, x: torch.Tensor, cache: KVCache, start: int, cos, sin) -> torch.Tensor:
        B, T, _ = x.shape
        H, Hk, d = self.H, self.H_kv, self.d
        q = self.q_norm(self.q(x).view(B, T, H, d)).transpose(1, 2)
        k = self.k_norm(self.k(x).view(B, T, Hk, d)).transpose(1, 2)
        v = self.v(x).view(B, T, Hk, d).transpose(1, 2)
        q, k = apply_rope(q, k, cos, sin)
        kc, vc = cache.k[self.layer_idx], cache.v[self.layer_idx]
        kc[:, :, start:start + T] = k
        vc[:, :, start:start + T] = v
        n = start + T
        if T == 1 and self.decode_attn_op is not None:
            if B != 1:
                raise ValueError("the decode seam takes batch 1 (use the graph decoder for batches)")
            out = self.decode_attn_op(q, kc[:, :, :n], vc[:, :, :n], scale=1.0 / math.sqrt(d),
                                      layer_idx=self.layer_idx)
        elif T == 1 and q.is_cuda:
            from .labeled_attn import dense_attention
            out = dense_attention(q[:, :, 0].reshape(B * H, d).contiguous(), kc.view(B * Hk, -1, d),
                                  vc.view(B * Hk, -1, d), n=n).view(B, H, 1, d)
        else:
            out = causal_attention(q, kc, vc, start)
        return self.o(out.transpose(1, 2).reshape(B, T, H * d))


class MLP(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.gate = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.up = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.down = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x):
        return self.down(torch.nn.functional.silu(self.gate(x)) * self.up(x))


class Layer(nn.Module):
    def __init__(self, cfg: Qwen3Config, i: int):
        super().__init__()
        self.norm1 = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.attn = Attention(cfg, i)
        self.norm2 = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.ffn = MLP(cfg)


class Qwen3Model(nn.Module):
    def __init__(self, cfg: Qwen3Config = QWEN3_0_6B):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(Layer(cfg, i) for i in range(cfg.num_hidden_layers))
        self.final_norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.lm_head = None if cfg.tie_word_embeddings else nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        cos, sin = rope_tables(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    def alloc_cache(self, max_len: int, batch: int = 1) -> KVCache:
        p = next(self.parameters())
        return KVCache(self.cfg, max_len, batch, p.dtype, p.device)

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        h = self.final_norm(h)
        return h @ self.embed.weight.T if self.lm_head is None else self.lm_head(h)

    def forward(self, ids: torch.Tensor, cache: KVCache, start_pos: int | None = None, *,
                last_only: bool = False) -> torch.Tensor:
        """Run ``ids [B, T]`` at positions ``start_pos ..`` (default: the cache's length), writing
        their keys and values; returns logits ``[B, T, vocab]`` (``[B, 1, vocab]`` with
        ``last_only``)."""
        start = cache.cur_len if start_pos is None else start_pos
        T = ids.shape[1]
        if start + T > cache.max_seq_len:
            raise ValueError("the cache is full")
        cos, sin = self.rope_cos[start:start + T], self.rope_sin[start:start + T]
        h = self.embed(ids)
        for layer in self.layers:
            h = h + layer.attn(layer.norm1(h), cache, start, cos, sin)
            h = h + layer.ffn(layer.norm2(h))
        cache.cur_len = start + T
        return self.logits(h[:, -1:] if last_only else h)


def random_model(cfg: Qwen3Config = QWEN3_0_6B, *, seed: int = 0, dtype=torch.bfloat16, device="cpu",
                 std: float = 0.02) -> Qwen3Model:
    """Random-init weights (normal with ``std``, norms at one) drawn on ``device`` from a seeded
    generator, as the benchmarks use (there is no checkpoint); the rotary tables stay fp32."""
    with torch.device(device):
        m = Qwen3Model(cfg)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=g)
    cos, sin = m.rope_cos, m.rope_sin
    m = m.to(dtype=dtype)
    m.rope_cos, m.rope_sin = cos, sin
    return m.eval()
