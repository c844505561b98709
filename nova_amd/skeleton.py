"""Synthetic decoder with Qwen3-4B geometry and random weights, the caller of the int8 KV path.

It stands in for ``NovaForCausalLM`` (src/nova/model.py:183-215) and reproduces the caller
contract of ``LeanAttention.forward`` (src/nova/layers.py:99-162): q/k/v projection, q/k head
norms, RoPE, then either the int8 cache (``update`` + ``attend`` / ``attend_prefill``, or the
fused ``update_attend`` for one decode token) or the fp16 cache (``update`` + SDPA with the
additive mask). Each layer is ``LeanDecoderLayer`` (layers.py:177-218): pre-norm attention and,
when ``intermediate_size > 0``, the SwiGLU MLP ``LeanMLP`` (layers.py:165-174), each added to
the residual stream. No checkpoint is loaded: weights are seeded random tensors.

Two ways to run a layer:

- torch (default): projections, norms and lm_head are plain torch ops around the KV path;
- ``use_decode_kernels()``: a one-token decode step (batch 1, int8 cache) runs each layer as
  three launches of this package's HIP kernels: the attention block in one
  (``update_attend_block``: the input RMSNorm and qkv projection, the q/k head norms + RoPE,
  the append and the attention of the token, o_proj with the residual add), gate/up GEMV with
  SwiGLU and the post-attention RMSNorm, down GEMV with the residual add; the final RMSNorm is
  fused into the lm_head GEMV. ``use_decode_kernels(fused_qkv=False)`` splits the attention
  block into the qkv GEMV, the head norms + RoPE, ``update_attend`` and the o_proj GEMV (the
  same bits). The same fp16 roundings as the torch path, up to fp32 summation order.
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
    intermediate_size: int = 9728  # 0: attention-only layers
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
    def __init__(self, cfg: SkeletonConfig, layer_idx: int, **factory):
        super().__init__()
        self.cfg = cfg
        self.layer_idx = layer_idx
        self.head_dim = cfg.head_dim
        self.scaling = cfg.head_dim ** -0.5
        self.q_proj = nn.Linear(cfg.hidden_size, cfg.num_attention_heads * cfg.head_dim, bias=False, **factory)
        self.k_proj = nn.Linear(cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim, bias=False, **factory)
        self.v_proj = nn.Linear(cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim, bias=False, **factory)
        self.o_proj = nn.Linear(cfg.num_attention_heads * cfg.head_dim, cfg.hidden_size, bias=False, **factory)
        self.q_norm = nn.Parameter(torch.ones(cfg.head_dim, **factory))
        self.k_norm = nn.Parameter(torch.ones(cfg.head_dim, **factory))

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


class SkeletonMLP(nn.Module):
    """``down(silu(gate(x)) * up(x))`` (``LeanMLP``, src/nova/layers.py:165-174)."""

    def __init__(self, cfg: SkeletonConfig, **factory):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False, **factory)
        self.up_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False, **factory)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False, **factory)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


def _stack_linears(*lins: nn.Linear) -> torch.Tensor:
    """One ``[sum(out), in]`` weight holding the given layers' weights, which become views of it."""
    w = torch.cat([lin.weight.detach() for lin in lins]).contiguous()
    o = 0
    for lin in lins:
        n = lin.weight.shape[0]
        lin.weight.data = w[o:o + n]
        o += n
    return w


class SkeletonLayer(nn.Module):
    def __init__(self, cfg: SkeletonConfig, layer_idx: int, **factory):
        super().__init__()
        self.norm = nn.Parameter(torch.ones(cfg.hidden_size, **factory))
        self.attn = SkeletonAttention(cfg, layer_idx, **factory)
        self.eps = cfg.rms_eps
        self.mlp = SkeletonMLP(cfg, **factory) if cfg.intermediate_size else None
        self.post_norm = nn.Parameter(torch.ones(cfg.hidden_size, **factory)) if self.mlp is not None else None
        self.w_qkv: torch.Tensor | None = None
        self.w_gate_up: torch.Tensor | None = None

    def forward(self, h, cos, sin, mask, cache):
        h = h + self.attn(_rms(h, self.norm, self.eps), cos, sin, mask, cache)
        if self.mlp is not None:
            h = h + self.mlp(_rms(h, self.post_norm, self.eps))
        return h

    def stack_weights(self) -> None:
        """Stack q/k/v and gate/up into single weights (the Linear weights become views)."""
        if self.w_qkv is None:
            a = self.attn
            self.w_qkv = _stack_linears(a.q_proj, a.k_proj, a.v_proj)
            if self.mlp is not None:
                self.w_gate_up = _stack_linears(self.mlp.gate_proj, self.mlp.up_proj)

    def decode_kernels(self, h: torch.Tensor, cache, pos: torch.Tensor, inv_freq: torch.Tensor,
                       fused_qkv: bool = True) -> torch.Tensor:
        """One decode token (``h`` of ``hidden_size`` elements) through the layer on the HIP
        kernels; returns the new residual stream (a new tensor). With ``fused_qkv`` (and a cache
        that has it) the projection, head norms, RoPE, attention step, o_proj and residual add are
        one launch (``update_attend_block``), bit for bit the same as the separate launches."""
        from . import gemv as G

        cfg, a = self.attn.cfg, self.attn
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        x = h.reshape(-1)
        if fused_qkv and hasattr(cache, "update_attend_block") and hq // hkv <= 4 and x.numel() % 8 == 0 \
                and x.numel() <= 3072 and hq * d <= 4096:
            # the projection, the head norms + RoPE, the attention step, o_proj and the residual
            # add in one launch
            h1 = cache.update_attend_block(x, self.w_qkv, self.norm, self.eps, a.q_norm, a.k_norm, cfg.rms_eps,
                                           inv_freq, a.o_proj.weight, a.layer_idx)
            if self.mlp is not None:
                act = G.swiglu_gemv(h1, self.w_gate_up, self.post_norm, self.eps)
                G.rms_gemv(act, self.mlp.down_proj.weight, residual=h1, out=h1)
            return h1.view(h.shape)
        if fused_qkv and hasattr(cache, "update_attend_qkv") and hq // hkv <= 4 and x.numel() % 8 == 0 \
                and x.numel() <= 3072:
            # the projection, the head norms + RoPE and the attention step in one launch
            o = cache.update_attend_qkv(x, self.w_qkv, self.norm, self.eps, a.q_norm, a.k_norm, cfg.rms_eps,
                                        inv_freq, a.layer_idx)
        else:
            qkv = G.rms_gemv(x, self.w_qkv, self.norm, self.eps)
            G.qk_norm_rope_(qkv, hq, hkv, a.q_norm, a.k_norm, cfg.rms_eps, inv_freq, pos)
            q = qkv[:hq * d].view(1, hq, 1, d)
            k = qkv[hq * d:(hq + hkv) * d].view(1, hkv, 1, d)
            v = qkv[(hq + hkv) * d:].view(1, hkv, 1, d)
            o = cache.update_attend(k, v, q, a.layer_idx)
        h1 = G.rms_gemv(o.reshape(-1), a.o_proj.weight, residual=x)
        if self.mlp is not None:
            act = G.swiglu_gemv(h1, self.w_gate_up, self.post_norm, self.eps)
            G.rms_gemv(act, self.mlp.down_proj.weight, residual=h1, out=h1)
        return h1.view(h.shape)


class SkeletonText(nn.Module):
    def __init__(self, cfg: SkeletonConfig, **factory):
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size, **factory)
        self.layers = nn.ModuleList([SkeletonLayer(cfg, i, **factory) for i in range(cfg.num_hidden_layers)])
        self.norm = nn.Parameter(torch.ones(cfg.hidden_size, **factory))
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float32) / cfg.head_dim))
        self.register_buffer("inv_freq", inv.to(factory.get("device")), persistent=False)
        # kernel mode: one-token steps over an int8 cache run on the HIP kernels, and the final
        # RMSNorm moves into the lm_head (``forward`` then returns the pre-norm hidden states)
        self.decode_kernels = False
        self.fused_qkv = True

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
        if self.decode_kernels:
            if (b == 1 and n == 1 and hasattr(past_key_values, "update_attend")
                    and not getattr(past_key_values, "prefilling", False)):
                h = self.embed_tokens(input_ids)
                pos = position_ids.reshape(-1)[:1]
                for layer in self.layers:
                    h = layer.decode_kernels(h, past_key_values, pos, self.inv_freq32, self.fused_qkv)
                return h
            return self._layers_torch(input_ids, position_ids, attention_mask, past_key_values)
        return _rms(self._layers_torch(input_ids, position_ids, attention_mask, past_key_values), self.norm,
                    self.cfg.rms_eps)

    def _layers_torch(self, input_ids, position_ids, attention_mask, past_key_values):
        freqs = position_ids.float()[..., None] * self.inv_freq  # [B, n, D/2]
        emb = torch.cat((freqs, freqs), dim=-1)[:, None]  # [B, 1, n, D]
        h = self.embed_tokens(input_ids)
        cos, sin = emb.cos().to(h.dtype), emb.sin().to(h.dtype)
        for layer in self.layers:
            h = layer(h, cos, sin, attention_mask, past_key_values)
        return h


class SkeletonForCausalLM(nn.Module):
    """Random-weight decoder: weights ~ N(0, 1) / sqrt(fan_in), norms 1.

    With ``device`` unset it is built in fp32 on the CPU from ``torch.Generator().manual_seed(seed)``
    (move it with ``.half().cuda()``); with ``device`` (and ``dtype``) it is built there
    directly, from a generator of that device, which a 4B-parameter geometry needs."""

    def __init__(self, cfg: SkeletonConfig | None = None, seed: int = 0, device=None, dtype: torch.dtype | None = None):
        super().__init__()
        cfg = cfg or SkeletonConfig()
        self.config = cfg
        factory = {} if device is None else {"device": torch.device(device), "dtype": dtype or torch.float16}
        self.model = SkeletonText(cfg, **factory)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False, **factory)
        g = torch.Generator(device=factory.get("device", "cpu")).manual_seed(seed)
        with torch.no_grad():
            for p in self.parameters():
                if p.dim() >= 2:
                    r = torch.randn(p.shape, generator=g, device=p.device, dtype=torch.float32)
                    p.copy_(r.mul_(p.shape[-1] ** -0.5))
                    del r

    def use_decode_kernels(self, on: bool = True, fused_qkv: bool = True) -> "SkeletonForCausalLM":
        """Run one-token decode steps on the HIP kernels (fp16 CUDA model, int8 cache); with
        ``fused_qkv`` each layer's projection, head norms, RoPE and attention step are one launch."""
        self.model.fused_qkv = bool(fused_qkv)
        if on:
            w = self.lm_head.weight
            if not w.is_cuda or w.dtype != torch.float16:
                raise ValueError("use_decode_kernels() needs the model in fp16 on the GPU")
            for layer in self.model.layers:
                layer.stack_weights()
            # the RoPE frequencies as the torch path promotes them (fp16 after ``.half()``)
            self.model.inv_freq32 = self.model.inv_freq.float().contiguous()
        self.model.decode_kernels = bool(on)
        return self

    def lm_head_forward(self, hidden: torch.Tensor) -> torch.Tensor:
        if not self.model.decode_kernels:
            return self.lm_head(hidden)
        # kernel mode: ``hidden`` is pre-norm; the final RMSNorm is part of the lm_head
        if hidden.shape[:-1].numel() == 1:
            from . import gemv as G

            logits = G.rms_gemv(hidden.reshape(-1), self.lm_head.weight, self.model.norm, self.config.rms_eps)
            return logits.view(*hidden.shape[:-1], -1)
        return self.lm_head(_rms(hidden, self.model.norm, self.config.rms_eps))

    def forward(self, input_ids, past_key_values=None, attention_mask=None, window_mask=None,
                cross_mode: str = "off", logits_to_keep: int = 0, position_ids=None):
        h = self.model(input_ids, past_key_values=past_key_values, position_ids=position_ids,
                       attention_mask=attention_mask, window_mask=window_mask, cross_mode=cross_mode)
        if logits_to_keep:
            h = h[:, -logits_to_keep:]
        return self.lm_head_forward(h)
