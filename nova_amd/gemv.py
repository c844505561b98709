"""Batch-1 decode-step projections of the synthetic decoder, on the HIP kernels of
``libnova_kv.so`` (``nkv_gemv``, ``nkv_swiglu_gemv``, ``nkv_qk_norm_rope``).

They fuse what a decoder layer runs around the int8 KV path for one token: the RMSNorm
(src/nova/norm.py:35-41) into the projection that reads its output, the residual add into
the projection that produces it, SwiGLU (``LeanMLP``, src/nova/layers.py:173-174) into the
gate/up projection, and the q/k head norms plus RoPE into one launch. Each function takes
fp16 CUDA tensors and the caller's preallocated ``out`` (graph capture), and raises when
the library is missing: there is no torch fallback here.
"""

from __future__ import annotations

import torch

from . import _lib


def _vec(t: torch.Tensor, name: str, n: int | None = None) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float16 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous fp16 CUDA tensor")
    if n is not None and t.numel() != n:
        raise ValueError(f"{name} has {t.numel()} elements, expected {n}")


def rms_gemv(x: torch.Tensor, w: torch.Tensor, gamma: torch.Tensor | None = None, eps: float = 1e-6,
             residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``W @ rms_norm(x) (+ residual)`` for one token: ``x`` has ``in`` elements, ``w`` is
    ``[out, in]``; the result has ``out`` elements and the shape of ``residual`` (when given)
    or ``x.shape[:-1] + (out,)``. ``gamma=None`` skips the norm. ``out`` may be ``residual``."""
    if w.dim() != 2:
        raise ValueError("w must be [out_features, in_features]")
    n_out, n_in = w.shape
    _vec(x, "x", n_in)
    _vec(w, "w")
    if gamma is not None:
        _vec(gamma, "gamma", n_in)
    if residual is not None:
        _vec(residual, "residual", n_out)
    if out is None:
        out = torch.empty(residual.shape if residual is not None else (*x.shape[:-1], n_out), dtype=x.dtype,
                          device=x.device)
    _vec(out, "out", n_out)
    if out.data_ptr() == x.data_ptr():
        raise ValueError("out must not alias x")
    _lib.call("nkv_gemv", x.data_ptr(), _lib.ptr(gamma), float(eps), w.data_ptr(), n_out, n_in, _lib.ptr(residual),
              out.data_ptr(), _lib.stream_ptr(x.device))
    return out


def swiglu_gemv(x: torch.Tensor, w_gate_up: torch.Tensor, gamma: torch.Tensor | None = None, eps: float = 1e-6,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(G @ xn) * (U @ xn)`` for one token with ``w_gate_up = cat([G, U])`` of
    ``[2 * intermediate, in]`` and ``xn = rms_norm(x)`` (``gamma=None``: ``x``)."""
    if w_gate_up.dim() != 2 or w_gate_up.shape[0] % 2:
        raise ValueError("w_gate_up must be [2 * intermediate, in_features]")
    inter, n_in = w_gate_up.shape[0] // 2, w_gate_up.shape[1]
    _vec(x, "x", n_in)
    _vec(w_gate_up, "w_gate_up")
    if gamma is not None:
        _vec(gamma, "gamma", n_in)
    if out is None:
        out = torch.empty((*x.shape[:-1], inter), dtype=x.dtype, device=x.device)
    _vec(out, "out", inter)
    _lib.call("nkv_swiglu_gemv", x.data_ptr(), _lib.ptr(gamma), float(eps), w_gate_up.data_ptr(), inter, n_in,
              out.data_ptr(), _lib.stream_ptr(x.device))
    return out


def qk_norm_rope_(qkv: torch.Tensor, hq: int, hkv: int, q_gamma: torch.Tensor, k_gamma: torch.Tensor,
                  eps: float, inv_freq: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """In place on one token's ``qkv`` (``(hq + 2 hkv) * 128`` elements, q then k then v heads):
    per-head RMSNorm of q and k, then RoPE at the device position ``pos`` (int64, one element)
    with ``inv_freq`` (fp32, 64 elements). Returns ``qkv``."""
    d = 128
    _vec(qkv, "qkv", (hq + 2 * hkv) * d)
    _vec(q_gamma, "q_gamma", d)
    _vec(k_gamma, "k_gamma", d)
    if inv_freq.dtype != torch.float32 or not inv_freq.is_contiguous() or inv_freq.numel() != d // 2:
        raise ValueError("inv_freq must be a contiguous fp32 tensor of 64 elements")
    if pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError("pos must be a one-element int64 tensor")
    _lib.call("nkv_qk_norm_rope", qkv.data_ptr(), hq, hkv, d, q_gamma.data_ptr(), k_gamma.data_ptr(), float(eps),
              inv_freq.data_ptr(), pos.data_ptr(), _lib.stream_ptr(qkv.device))
    return qkv
