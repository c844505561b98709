"""Per-token symmetric int8 KV format ("tok") on MI355X.

An extension beside the reference's ``int8t64`` format (src/nova/kvquant.py:118-176,
src/nova/kvattn.py:488-880): one symmetric absmax scale per (token, KV head) row of 128,
fp16 scales, int8 codes. Rounding follows kvquant's conventions:

    scale = max(max|x| / 127, 1e-8)   (fp32; stored as fp16)
    code  = clamp(rint(x / scale), -127, 127)   (with the fp32 scale)
    value = fp16(code * scale16)

A token is quantized once, when it is written, so a cache in this format keeps every
token as int8 (no fp16 ring, no requantization) and reads 2080 bytes per token and layer
over 8 KV heads. Every computation runs in the HIP kernels of ``libnova_kv.so``.

- :func:`quantize_tok` / :func:`dequantize_tok`: the quantizer and its inverse.
- :func:`int8_tok_attn_decode`: decode attention over a tok cache (split-K, two launches).
- :class:`KVInt8TokCache`: the streaming cache with the decode-loop surface of
  ``KVInt8Cache`` (``update`` / ``attend`` / ``update_attend`` / ``finish_prefill``).
"""

from __future__ import annotations

import torch

from . import _lib
from .kvquant import _DT, _on_gpu, _prep

D = 128
GROUP = 64  # capacity granularity (one streamed group)


def quantize_tok(x: torch.Tensor):
    """``x`` ``[..., n, 128]`` (fp16 / bf16 / fp32, on the GPU) -> ``(int8 [..., n, 128], fp16 [..., n])``."""
    _on_gpu(x, "x")
    if x.dtype not in _DT:
        raise ValueError(f"unsupported dtype {x.dtype}")
    if x.shape[-1] != D:
        raise NotImplementedError(f"head_dim {x.shape[-1]}: the HIP kernels are built for {D}")
    *lead, n, dim = x.shape
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty((*lead, n), dtype=torch.float16, device=x.device)
    if x.numel() == 0:
        return q, s
    xc, rows, rs = _prep(x)
    _lib.call("nkv_quantize_tok", xc.data_ptr(), _DT[x.dtype], rs, rows, n, dim, q.data_ptr(), n * dim,
              s.data_ptr(), n, _lib.stream_ptr(x.device))
    return q, s


def dequantize_tok(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Inverse of :func:`quantize_tok`: ``code * scale16`` rounded once to ``dtype``."""
    _on_gpu(q, "q")
    if q.dtype != torch.int8 or scale.dtype != torch.float16:
        raise ValueError("q must be int8 and scale fp16")
    if q.shape[-1] != D or scale.shape != q.shape[:-1]:
        raise ValueError(f"shapes {tuple(q.shape)} / {tuple(scale.shape)} do not match")
    *lead, n, dim = q.shape
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    if q.numel() == 0:
        return out
    qc, sc = q.contiguous(), scale.contiguous()
    rows = qc.numel() // (n * dim)
    _lib.call("nkv_dequantize_tok", qc.data_ptr(), n * dim, sc.data_ptr(), n, rows, n, dim, out.data_ptr(),
              _DT[dtype], n * dim, _lib.stream_ptr(q.device))
    return out


def _check(x: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not x.is_cuda:
        raise ValueError(f"{name} must be on the GPU")
    if x.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _parts(hkv: int, hq: int, groups: int, ws_bytes: int) -> int:
    lib = _lib.load()
    parts = int(lib.nkv_attn_default_parts(hkv, groups))
    per_part = int(lib.nkv_attn_workspace_bytes(hkv, hq, 1))
    return max(1, min(parts, ws_bytes // per_part))


def int8_tok_attn_decode(q: torch.Tensor, kq: torch.Tensor, ksc: torch.Tensor, vq: torch.Tensor,
                         vsc: torch.Tensor, *, used: int | None = None, used_t: torch.Tensor | None = None,
                         out: torch.Tensor | None = None, lse_out: torch.Tensor | None = None,
                         scratch: torch.Tensor | None = None, n_splits: int | None = None) -> torch.Tensor:
    """Decode attention over tokens ``[0, used)`` of a tok cache.

    ``q`` fp16 ``[1, Hq, 1, 128]``; ``kq``/``vq`` int8 ``[1, Hkv, L, 128]`` with ``L`` a
    multiple of 64; ``ksc``/``vsc`` fp16 ``[1, Hkv, L]``. ``used`` (host int) or
    ``used_t`` (device int64 ``[1]``, graph-safe) gives the length; ``out`` / ``lse_out``
    / ``scratch`` may be preallocated for capture. Returns ``out`` ``[1, Hq, 1, 128]``.
    """
    _check(q, "q", torch.float16)
    for t, nm in ((kq, "kq"), (vq, "vq")):
        _check(t, nm, torch.int8)
    for t, nm in ((ksc, "ksc"), (vsc, "vsc")):
        _check(t, nm, torch.float16)
    if q.shape[0] != 1 or q.shape[2] != 1:
        raise ValueError("batch 1, one decode token (解码一步)")
    _, hq, _, d = q.shape
    _, hkv, cap, _ = kq.shape
    if used_t is None:
        used = cap if used is None else int(used)
        if not 0 <= used <= cap:
            raise ValueError(f"used={used} outside [0, {cap}]")
    if out is None:
        out = torch.empty_like(q)
    groups = cap // GROUP
    if scratch is None:
        parts = int(n_splits) if n_splits else int(_lib.load().nkv_attn_default_parts(hkv, groups))
        scratch = _lib.workspace(q.device, int(_lib.load().nkv_attn_workspace_bytes(hkv, hq, parts)), "decode")
    else:
        parts = int(n_splits) if n_splits else _parts(hkv, hq, groups, scratch.numel() * scratch.element_size())
    _lib.call("nkv_attn_decode_tok", q.data_ptr(), kq.data_ptr(), ksc.data_ptr(), vq.data_ptr(), vsc.data_ptr(),
              hq, hkv, d, cap, 0 if used_t is not None else used, _lib.ptr(used_t), out.data_ptr(),
              _lib.ptr(lse_out), scratch.data_ptr(), scratch.numel() * scratch.element_size(), parts,
              _lib.stream_ptr(q.device))
    return out


class KVInt8TokCache:
    """Streaming int8 KV cache in the per-token symmetric format.

    The decode-loop surface mirrors ``KVInt8Cache`` (src/nova/kvattn.py:488-880):
    device scalars ``pos`` and ``_written``, ``update`` / ``attend`` / ``update_attend``
    per layer, ``set_prefill_pos`` + ``update`` of a chunk + ``finish_prefill`` for the
    prompt. Every token is stored as int8 when written, so there is no fp16 ring and no
    staging area: a prefill chunk is quantized straight into the cache.
    """

    def __init__(self, num_slots: int, num_kv_heads: int, head_dim: int, max_len: int, num_q_heads: int,
                 batch: int = 1, dtype: torch.dtype = torch.float16, device: str | torch.device = "cuda") -> None:
        if head_dim != D or dtype != torch.float16:
            raise NotImplementedError("the HIP path stores fp16 K/V with head_dim 128")
        if num_q_heads % num_kv_heads or num_q_heads // num_kv_heads > 16:
            raise ValueError(f"Q heads {num_q_heads} / KV heads {num_kv_heads}")
        if batch != 1:
            raise ValueError("batch 必须为 1")
        _lib.load()
        self.num_slots, self.num_kv_heads, self.head_dim = int(num_slots), int(num_kv_heads), int(head_dim)
        self.num_q_heads, self.batch, self.dtype, self.device = int(num_q_heads), int(batch), dtype, device
        self.max_len = -(-int(max_len) // GROUP) * GROUP  # capacity: a multiple of 64
        dshape = (1, self.num_kv_heads, self.max_len, self.head_dim)
        sshape = (1, self.num_kv_heads, self.max_len)
        self.kq = [torch.zeros(dshape, dtype=torch.int8, device=device) for _ in range(self.num_slots)]
        self.vq = [torch.zeros(dshape, dtype=torch.int8, device=device) for _ in range(self.num_slots)]
        self.ksc = [torch.zeros(sshape, dtype=dtype, device=device) for _ in range(self.num_slots)]
        self.vsc = [torch.zeros(sshape, dtype=dtype, device=device) for _ in range(self.num_slots)]
        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        self._written = torch.zeros(1, dtype=torch.long, device=device)
        self._prefill_off = 0
        self._n_parts = int(_lib.load().nkv_attn_default_parts(self.num_kv_heads, self.max_len // GROUP))
        self._ws_bytes = int(_lib.load().nkv_attn_workspace_bytes(self.num_kv_heads, self.num_q_heads, self._n_parts))
        self.pa = torch.zeros(self._ws_bytes // 4, dtype=torch.float32, device=device)
        self.lse = torch.zeros((1, self.num_q_heads), dtype=torch.float32, device=device)
        self.merged = torch.zeros((1, self.num_q_heads, 1, self.head_dim), dtype=dtype, device=device)

    def set_parts(self, n_parts: int) -> None:
        """Prefix work units per KV head for the decode launches (before any capture); grows
        the zero-filled workspace when needed."""
        need = int(_lib.load().nkv_attn_workspace_bytes(self.num_kv_heads, self.num_q_heads, int(n_parts)))
        if need > self._ws_bytes:
            self._ws_bytes = need
            self.pa = torch.zeros(need // 4, dtype=torch.float32, device=self.pa.device)
        self._n_parts = int(n_parts)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self.pos.item())

    def reset(self) -> None:
        self.pos.zero_()
        self._written.zero_()
        self._prefill_off = 0

    # ---- prefill: chunks quantized straight into the cache

    def set_prefill_pos(self, off: int) -> None:
        self._prefill_off = int(off)
        self.pos.fill_(int(off))

    def update(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int):
        """Write K/V. During a prefill (``begin_prefill``) a chunk of n tokens is quantized
        straight into ``[off, off + n)``, ``off`` from ``set_prefill_pos``; otherwise one
        decode token is appended at ``pos`` (device scalar, graph-safe)."""
        n = key.shape[2]
        if self._in_prefill:
            off = self._prefill_off
            if off + n > self.max_len:
                raise ValueError(f"prefill [{off}, {off + n}) exceeds the capacity {self.max_len}")
            for src, dq, ds in ((key, self.kq[layer_idx], self.ksc[layer_idx]),
                                (value, self.vq[layer_idx], self.vsc[layer_idx])):
                if src.shape != (1, self.num_kv_heads, n, self.head_dim) or src.dtype not in _DT:
                    raise ValueError(f"prefill chunk must be [1, {self.num_kv_heads}, n, {self.head_dim}]")
                x, rows, rs = _prep(src)
                _lib.call("nkv_quantize_tok", x.data_ptr(), _DT[src.dtype], rs, rows, n, self.head_dim,
                          dq[0, 0, off:].data_ptr(), self.max_len * self.head_dim, ds[0, 0, off:].data_ptr(),
                          self.max_len, _lib.stream_ptr(self.pos.device))
            return None, None
        if n != 1:
            raise RuntimeError("没有 prefill 时只支持解码一步（n == 1）；prefill 请先 `begin_prefill()`")
        k, v = self._token(key, "key"), self._token(value, "value")
        _lib.call("nkv_append_tok", k.data_ptr(), v.data_ptr(), k.stride(1), self.kq[layer_idx].data_ptr(),
                  self.ksc[layer_idx].data_ptr(), self.vq[layer_idx].data_ptr(), self.vsc[layer_idx].data_ptr(),
                  self.pos.data_ptr(), self._written.data_ptr(), self.num_kv_heads, self.head_dim, self.max_len,
                  _lib.stream_ptr(self.pos.device))
        return None, None

    append_prefill = update
    _in_prefill = False

    def begin_prefill(self, total_len: int) -> None:
        if not 0 < int(total_len) <= self.max_len:
            raise ValueError(f"prefill 长度 {total_len} 超出 (0, {self.max_len}]")
        self._in_prefill = True
        self._prefill_off = 0

    def finish_prefill(self, total: int) -> None:
        """End the prompt: ``pos = written = total``."""
        self.pos.fill_(int(total))
        self._written.fill_(int(total))
        self._in_prefill = False

    def _token(self, x: torch.Tensor, name: str) -> torch.Tensor:
        if x.shape != (1, self.num_kv_heads, 1, self.head_dim) or x.dtype != self.dtype:
            raise ValueError(f"{name} must be fp16 [1, {self.num_kv_heads}, 1, {self.head_dim}], got "
                             f"{tuple(x.shape)} {x.dtype}")
        if x.stride(3) != 1 or x.stride(1) % 8 or x.data_ptr() % 16:
            x = x.contiguous()
        return x

    def _q(self, query: torch.Tensor) -> torch.Tensor:
        if query.shape != (1, self.num_q_heads, 1, self.head_dim) or query.dtype != self.dtype:
            raise ValueError(f"query must be fp16 [1, {self.num_q_heads}, 1, {self.head_dim}] (解码一步), got "
                             f"{tuple(query.shape)} {query.dtype}")
        return query if query.is_contiguous() and query.data_ptr() % 16 == 0 else query.contiguous()

    # ---- decode

    def attend(self, query: torch.Tensor, layer_idx: int) -> torch.Tensor:
        """Attention over ``[0, _written)`` of layer ``layer_idx`` (two HIP launches)."""
        q = self._q(query)
        _lib.call("nkv_attn_decode_tok", q.data_ptr(), self.kq[layer_idx].data_ptr(), self.ksc[layer_idx].data_ptr(),
                  self.vq[layer_idx].data_ptr(), self.vsc[layer_idx].data_ptr(), self.num_q_heads,
                  self.num_kv_heads, self.head_dim, self.max_len, 0, self._written.data_ptr(),
                  self.merged.data_ptr(), self.lse.data_ptr(), self.pa.data_ptr(), self._ws_bytes, self._n_parts,
                  _lib.stream_ptr(self.pos.device))
        return self.merged

    def _output(self, out: torch.Tensor | None) -> torch.Tensor:
        if out is None:
            return self.merged
        if (tuple(out.shape) != tuple(self.merged.shape) or out.dtype != self.dtype or not out.is_contiguous()
                or out.data_ptr() % 16 or out.device != self.merged.device):
            raise ValueError(f"out must be a contiguous, 16-byte aligned {self.dtype} tensor of shape "
                             f"{tuple(self.merged.shape)} on {self.merged.device}")
        return out

    def step_args(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer_idx: int,
                  out: torch.Tensor | None = None) -> tuple:
        """Arguments of ``nkv_decode_step_tok`` for one decode token of ``layer_idx``."""
        k, v, q = self._token(key, "key"), self._token(value, "value"), self._q(query)
        o = self._output(out)
        return (q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(1), self.kq[layer_idx].data_ptr(),
                self.ksc[layer_idx].data_ptr(), self.vq[layer_idx].data_ptr(), self.vsc[layer_idx].data_ptr(),
                self.pos.data_ptr(), self._written.data_ptr(), self.num_q_heads, self.num_kv_heads, self.head_dim,
                self.max_len, o.data_ptr(), self.lse.data_ptr(), self.pa.data_ptr(), self._ws_bytes,
                self._n_parts, _lib.stream_ptr(self.pos.device))

    def update_attend(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer_idx: int,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """Append of the token at ``pos`` + attention over ``[0, pos]`` in one launch; the output
        goes to ``out`` when given, else to ``merged``."""
        _lib.call("nkv_decode_step_tok", *self.step_args(key, value, query, layer_idx, out))
        return self._output(out)

    def nbytes(self) -> int:
        """Resident KV bytes: codes and scales."""
        return sum(t.numel() * t.element_size() for t in self.kq + self.vq + self.ksc + self.vsc)
