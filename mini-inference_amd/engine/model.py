"""Qwen2 decoder used as the harness around the paged KV-cache kernels.

The attention layer hands its post-RoPE q, k, v to an ``AttentionContext`` and gets the
attention output back, exactly as engine/model.py:241-251 of the reference does
(``out = ctx.attend(self.layer_idx, q, k, v)``). The cache contexts in
:mod:`engine.kv_cache` implement that protocol with the HIP kernels; this module only
supplies the surrounding projections, norms, RoPE and MLP in PyTorch so that a full
decode step can be timed with random-init weights (no checkpoint is loaded).

Shapes (reference engine/model.py:89-98): q ``[B, Hq, T, D]``, k and v
``[B, Hkv, T, D]``; ``attend`` returns ``[B, Hq, T, D]``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Protocol

import torch
import torch.nn.functional as F
from torch import nn


@dataclass(frozen=True)
class Qwen2Config:
    """Architecture numbers (field names as engine/model.py:37-86)."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_position_embeddings: int = 32768
    tie_word_embeddings: bool = True
    attention_bias: bool = True

    @property
    def q_size(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim

    @classmethod
    def qwen2_5_0_5b(cls) -> "Qwen2Config":
        """Qwen2.5-0.5B: 24 layers, hidden 896, 14 query / 2 KV heads of 64, tied embeddings."""
        return cls(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_layers=24, num_heads=14,
                   num_kv_heads=2, head_dim=64)

    @classmethod
    def qwen2_7b_like(cls) -> "Qwen2Config":
        """The 7B-class GQA shape: 28 layers, 28 query / 4 KV heads of 128."""
        return cls(vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_layers=28, num_heads=28,
                   num_kv_heads=4, head_dim=128, tie_word_embeddings=False)


class AttentionContext(Protocol):
    """Receives one layer's post-RoPE q, k, v; stores k/v; returns attention output.

    A context whose ``fuse_rope`` attribute is true instead receives q and k before the
    rotary embedding, with the step's cos/sin tables, through
    ``attend_rope(layer_idx, q, k, v, cos, sin)``, and applies the rotation itself.
    """

    def attend(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor: ...


class RMSNorm(nn.Module):
    """x / rms(x) * weight with the statistic taken in fp32, result cast back first."""

    def __init__(self, dim: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + self.eps)
        return self.weight * (xf * inv).to(x.dtype)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype: torch.dtype):
    """cos/sin ``[B, 1, T, D]`` for per-token ``positions [B, T]`` (half-rotation layout)."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(half, device=positions.device, dtype=torch.float32) * 2.0 / head_dim))
    ang = positions.to(torch.float32).unsqueeze(-1) * inv_freq  # [B, T, D/2]
    ang = torch.cat((ang, ang), dim=-1).unsqueeze(1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    def rot(x: torch.Tensor) -> torch.Tensor:
        a, b = x.chunk(2, dim=-1)
        return torch.cat((-b, a), dim=-1)

    return q * cos + rot(q) * sin, k * cos + rot(k) * sin


class Attention(nn.Module):
    def __init__(self, cfg: Qwen2Config, layer_idx: int) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.cfg = cfg
        self.qkv_proj = nn.Linear(cfg.hidden_size, cfg.q_size + 2 * cfg.kv_size, bias=cfg.attention_bias)
        self.o_proj = nn.Linear(cfg.q_size, cfg.hidden_size, bias=False)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, ctx: AttentionContext) -> torch.Tensor:
        c = self.cfg
        bsz, t, _ = x.shape
        q, k, v = self.qkv_proj(x).split([c.q_size, c.kv_size, c.kv_size], dim=-1)
        q = q.view(bsz, t, c.num_heads, c.head_dim).transpose(1, 2)
        k = k.view(bsz, t, c.num_kv_heads, c.head_dim).transpose(1, 2)
        v = v.view(bsz, t, c.num_kv_heads, c.head_dim).transpose(1, 2)
        if getattr(ctx, "fuse_rope", False):
            # The context rotates q and k itself (in place), fused with its KV append.
            out = ctx.attend_rope(self.layer_idx, q, k, v, cos, sin)
        else:
            q, k = apply_rope(q, k, cos, sin)
            out = ctx.attend(self.layer_idx, q, k, v)  # the call site the cache contexts serve
        return self.o_proj(out.transpose(1, 2).reshape(bsz, t, c.q_size))


class MLP(nn.Module):
    def __init__(self, cfg: Qwen2Config) -> None:
        super().__init__()
        self.gate_up_proj = nn.Linear(cfg.hidden_size, 2 * cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class DecoderLayer(nn.Module):
    def __init__(self, cfg: Qwen2Config, layer_idx: int) -> None:
        super().__init__()
        self.input_norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.attn = Attention(cfg, layer_idx)
        self.post_attn_norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.mlp = MLP(cfg)

    def forward(self, x, cos, sin, ctx):
        x = x + self.attn(self.input_norm(x), cos, sin, ctx)
        return x + self.mlp(self.post_attn_norm(x))


class Qwen2ForCausalLM(nn.Module):
    """Embedding -> decoder layers -> final norm; ``compute_logits`` applies the LM head."""

    def __init__(self, cfg: Qwen2Config) -> None:
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg, i) for i in range(cfg.num_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.lm_head = None if cfg.tie_word_embeddings else nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, ctx: AttentionContext) -> torch.Tensor:
        x = self.embed_tokens(input_ids)
        cos, sin = rope_cos_sin(positions, self.cfg.head_dim, self.cfg.rope_theta, x.dtype)
        for layer in self.layers:
            x = layer(x, cos, sin, ctx)
        return self.norm(x)

    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        w = self.embed_tokens.weight if self.lm_head is None else self.lm_head.weight
        return F.linear(hidden, w)


def random_init_(model: Qwen2ForCausalLM, seed: int = 0, std: float = 0.02) -> Qwen2ForCausalLM:
    """Fill every weight in place from a seeded normal on its own device (norm weights stay 1)."""
    dev = next(model.parameters()).device
    gen = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=gen)
    return model


def head_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
