"""Synthetic attention-only decoder with Qwen3-4B attention geometry and random weights.

It stands in for ``NovaForCausalLM`` (src/nova/model.py:183-215) as the caller of the
int8 KV path, reproducing the caller contract of ``LeanAttention.forward``
(src/nova/layers.py:99-162): q/k/v projection, RoPE, then either the int8 cache
(``update`` + ``attend`` / ``attend_prefill``, or the fused ``update_attend`` for one
decode token) or the fp16 cache (``update`` + SDPA with the additive mask). Its
projections, norms and lm_head are plain torch ops — they sit outside the path.
No checkpoint is loaded: weights are seeded random tensors.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class SkeletonConfig:
    num_hidden_layers: int = 36
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    hidden_size: int = 2560
    vocab_size: int = 2048
    rope_theta: float = 1_000_000.0
    rms_eps: float = 1e-6

    @property
    def num_key_value_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``[B, H_kv, n, D]`` -> ``[B, H_kv * n_rep, n, D]`` (src/nova/layers.py:39-45)."""
    b, h, n, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None].expand(b, h, n_rep, n, d).reshape(b, h * n_rep, n, d)


class SkeletonAttention(nn.Module):
    def __init__(self, cfg: SkeletonConfig, layer_idx: int):
        super().__init__()
        self.cfg = cfg
        self.layer_idx = layer_idx
        self.head_dim = cfg.head_dim
        self.scaling = cfg.head_dim ** -0.5
        self.q_proj = nn.Linear(cfg.hidden_size, cfg.num_attention_heads * cfg.head_dim, bias=False)
        self.k_proj = nn.Linear(cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim, bias=False)
        self.v_proj = nn.Linear(cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim, bias=False)
        self.o_proj = nn.Linear(cfg.num_attention_heads * cfg.head_dim, cfg.hidden_size, bias=False)
        self.q_norm = nn.Parameter(torch.ones(cfg.head_dim))
        self.k_norm = nn.Parameter(torch.ones(cfg.head_dim))

    def forward(self, hidden: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                attention_mask: torch.Tensor | None, cache) -> torch.Tensor:
        b, n, _ = hidden.shape
        shp = (b, n, -1, self.head_dim)
        q = _rms(self.q_proj(hidden).view(shp), self.q_norm, self.cfg.rms_eps).transpose(1, 2)
        k = _rms(self.k_proj(hidden).view(shp), self.k_norm, self.cfg.rms_eps).transpose(1, 2)
        v = self.v_proj(hidden).view(shp).transpose(1, 2)
        q = q * cos + _rotate_half(q) * sin
        k = k * cos + _rotate_half(k) * sin
        if hasattr(cache, "attend"):
            # the int8 cache's caller contract (src/nova/layers.py:127-137)
            if n == 1 and not getattr(cache, "prefilling", False) and hasattr(cache, "update_attend"):
                out = cache.update_attend(k, v, q, self.layer_idx)
            else:
                cache.update(k, v, self.layer_idx)
                out = cache.attend_prefill(q, self.layer_idx) if n > 1 else cache.attend(q, self.layer_idx)
        else:
            k, v = cache.update(k, v, self.layer_idx)
            rep = self.cfg.num_key_value_groups
            k, v = repeat_kv(k, rep), repeat_kv(v, rep)
            is_causal = n > 1 and attention_mask is None
            if is_causal and k.shape[2] > n:
                k, v = k[:, :, :n], v[:, :, :n]
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=attention_mask, dropout_p=0.0,
                                                 scale=self.scaling, is_causal=is_causal)
        return self.o_proj(out.transpose(1, 2).reshape(b, n, -1).contiguous())


class SkeletonLayer(nn.Module):
    def __init__(self, cfg: SkeletonConfig, layer_idx: int):
        super().__init__()
        self.norm = nn.Parameter(torch.ones(cfg.hidden_size))
        self.attn = SkeletonAttention(cfg, layer_idx)
        self.eps = cfg.rms_eps

    def forward(self, h, cos, sin, mask, cache):
        return h + self.attn(_rms(h, self.norm, self.eps), cos, sin, mask, cache)


class SkeletonText(nn.Module):
    def __init__(self, cfg: SkeletonConfig):
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList([SkeletonLayer(cfg, i) for i in range(cfg.num_hidden_layers)])
        self.norm = nn.Parameter(torch.ones(cfg.hidden_size))
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float32) / cfg.head_dim))
        self.register_buffer("inv_freq", inv, persistent=False)

    @property
    def num_cache_layers(self) -> int:
        return self.cfg.num_hidden_layers

    @property
    def layer_windows(self) -> list[int]:
        return [0] * self.cfg.num_hidden_layers

    def forward(self, input_ids, past_key_values=None, position_ids=None, attention_mask=None,
                window_mask=None, cross_mode: str = "off"):
        b, n = input_ids.shape
        if position_ids is None:
            position_ids = past_key_values.pos.view(1, 1) + torch.arange(n, device=input_ids.device).view(1, n)
        elif position_ids.dim() == 3:  # [3, B, n] multimodal positions: the text axis
            position_ids = position_ids[0]
        freqs = position_ids.float()[..., None] * self.inv_freq  # [B, n, D/2]
        emb = torch.cat((freqs, freqs), dim=-1)[:, None]  # [B, 1, n, D]
        h = self.embed_tokens(input_ids)
        cos, sin = emb.cos().to(h.dtype), emb.sin().to(h.dtype)
        for layer in self.layers:
            h = layer(h, cos, sin, attention_mask, past_key_values)
        return _rms(h, self.norm, self.cfg.rms_eps)


class SkeletonForCausalLM(nn.Module):
    def __init__(self, cfg: SkeletonConfig | None = None, seed: int = 0):
        super().__init__()
        cfg = cfg or SkeletonConfig()
        self.config = cfg
        g = torch.Generator().manual_seed(seed)
        self.model = SkeletonText(cfg)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        with torch.no_grad():
            for p in self.parameters():
                if p.dim() >= 2:
                    p.copy_(torch.randn(p.shape, generator=g) * (p.shape[-1] ** -0.5))

    def lm_head_forward(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.lm_head(hidden)

    def forward(self, input_ids, past_key_values=None, attention_mask=None, window_mask=None,
                cross_mode: str = "off", logits_to_keep: int = 0, position_ids=None):
        h = self.model(input_ids, past_key_values=past_key_values, position_ids=position_ids,
                       attention_mask=attention_mask, window_mask=window_mask, cross_mode=cross_mode)
        if logits_to_keep:
            h = h[:, -logits_to_keep:]
        return self.lm_head_forward(h)
