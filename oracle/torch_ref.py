"""torch fp32 restatement of the reference's int8 decode step on the CPU — TEST INFRASTRUCTURE ONLY.

The benchmark's CPU baseline times this module on the host cores. It is the reference's own
algorithm for one decode step of one layer, as its tests compute it:

1. dequantize the int8t64 prefix with the stored fp16 rulers
   (``src/nova/kvquant.py:152-176``: ``fp16(fp32(q) * fp32(step16) + fp32(min16))``);
2. append the valid fp16 ring slots (``src/nova/kvattn.py:819-833``: slot ``i`` holds position
   ``u - ((u - i) mod 64)``, valid iff ``qlen <= p <= u`` and ``p >= first``);
3. expand the KV heads to the query heads (``repeat_kv``, ``src/nova/layers.py:39-45``) and
   run softmax attention in fp32 (``tests/test_kvattn.py:62-70``: the reference checks its
   kernel against ``dequantize_int8`` -> SDPA).

The per-token symmetric format dequantizes as ``fp16(fp32(code) * fp32(scale16))``.

``tests/test_oracle.py`` pins these functions against the numpy oracle (``oracle.attn``,
``oracle.stream``), which the reference's own vectors pin in turn.
"""

from __future__ import annotations

import torch

GROUP = 64


def dequantize_int8_token(q: torch.Tensor, mins: torch.Tensor, steps: torch.Tensor,
                          group: int = GROUP) -> torch.Tensor:
    """``q`` uint8 ``[..., n, D]``, rulers fp16 ``[..., ceil(n/group), D]`` -> fp16 ``[..., n, D]``
    (``src/nova/kvquant.py:167-176``: pad by repeating the last token, per-group affine map in
    fp32, round to fp16)."""
    n, d = q.shape[-2], q.shape[-1]
    pad = (-n) % group
    qf = q.float()
    if pad:
        qf = torch.cat([qf, qf[..., -1:, :].expand(*qf.shape[:-2], pad, d)], dim=-2)
    g = qf.reshape(*qf.shape[:-2], (n + pad) // group, group, d)
    x = g * steps.float().unsqueeze(-2) + mins.float().unsqueeze(-2)
    return x.reshape(*qf.shape[:-2], n + pad, d)[..., :n, :].to(torch.float16)


def dequantize_tok(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Per-token symmetric int8: ``fp16(fp32(code) * fp32(scale16))``; ``codes`` ``[..., n, D]``
    int8, ``scales`` ``[..., n]`` fp16."""
    return (codes.float() * scales.float().unsqueeze(-1)).to(torch.float16)


def ring_mask(written: int, qlen: int, first: int, slots: int = GROUP) -> torch.Tensor:
    """Valid ring slots (``src/nova/kvattn.py:819-833``) as a bool ``[slots]``."""
    u = written - 1
    i = torch.arange(slots)
    p = u - torch.remainder(u - i, slots)
    return (p >= qlen) & (p <= u) & (p >= first)


def attend(q: torch.Tensor, k16: torch.Tensor, v16: torch.Tensor) -> torch.Tensor:
    """Softmax attention of one decode token in fp32 with the KV heads repeated to the query
    heads. ``q`` ``[Hq, D]``, ``k16``/``v16`` ``[Hkv, n, D]`` -> fp16 ``[Hq, D]``."""
    hq, d = q.shape
    hkv = k16.shape[0]
    k = k16.float().repeat_interleave(hq // hkv, dim=0)
    v = v16.float().repeat_interleave(hq // hkv, dim=0)
    s = torch.bmm(k, q.float().unsqueeze(-1)).squeeze(-1) * d ** -0.5
    p = torch.softmax(s, dim=-1)
    return torch.bmm(p.unsqueeze(1), v).squeeze(1).to(torch.float16)


def decode_step_t64(q, kq, kmn, kst, vq, vmn, vst, tail_k, tail_v, written: int, first: int = 0):
    """One decode step of one layer of the streaming int8t64 cache: the int8 prefix
    ``[0, qlen)`` (``qlen = 64 * floor(written / 64)``) dequantized, the valid ring slots
    appended, then attention. Shapes as in the cache, batch axis dropped: ``kq`` ``[Hkv, L, D]``
    uint8, rulers ``[Hkv, ceil(L/64), D]`` fp16, ring ``[Hkv, 64, D]`` fp16, ``q`` ``[Hq, D]``."""
    qlen = written // GROUP * GROUP
    ng = qlen // GROUP
    k16 = dequantize_int8_token(kq[:, :qlen], kmn[:, :ng], kst[:, :ng])
    v16 = dequantize_int8_token(vq[:, :qlen], vmn[:, :ng], vst[:, :ng])
    m = ring_mask(written, qlen, first, tail_k.shape[1])
    k_all = torch.cat([k16, tail_k[:, m]], dim=1)
    v_all = torch.cat([v16, tail_v[:, m]], dim=1)
    return attend(q, k_all, v_all)


def decode_step_tok(q, kq, ks, vq, vs, used: int):
    """One decode step of one layer of the per-token symmetric cache over tokens ``[0, used)``."""
    return attend(q, dequantize_tok(kq[:, :used], ks[:, :used]), dequantize_tok(vq[:, :used], vs[:, :used]))
