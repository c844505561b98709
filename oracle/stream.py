"""numpy restatement of the streaming int8 KV cache state machine (checker only).

Follows ``KVInt8Cache`` in ``src/nova/kvattn.py:549-862`` step by step: an int8
prefix of whole 64-token groups, a 64-slot fp16 ring holding the newest tokens
(slot = absolute position mod 64), and three scalars derived from ``pos``.
"""

from __future__ import annotations

import numpy as np

from . import attn as oattn
from . import kvquant as okq


class StreamCache:
    """Per-layer state with the reference's shapes minus the batch axis (batch is 1).

    ``kq``/``vq`` [Hkv, max_len, D] uint8, rulers [Hkv, ceil(max_len/64), D] fp16,
    ``tail_k``/``tail_v`` [Hkv, 64, D] fp16 (``kvattn.py:589-601``).
    """

    def __init__(self, num_slots: int, num_kv_heads: int, head_dim: int, max_len: int,
                 num_q_heads: int, group: int = 64):
        self.num_slots, self.h, self.d = num_slots, num_kv_heads, head_dim
        self.max_len, self.hq, self.group = max_len, num_q_heads, group
        ng = -(-max_len // group)
        z8 = lambda: np.zeros((num_kv_heads, max_len, head_dim), np.uint8)  # noqa: E731
        z16 = lambda n: np.zeros((num_kv_heads, n, head_dim), np.float16)  # noqa: E731
        self.kq = [z8() for _ in range(num_slots)]
        self.vq = [z8() for _ in range(num_slots)]
        self.kmn = [z16(ng) for _ in range(num_slots)]
        self.kst = [z16(ng) for _ in range(num_slots)]
        self.vmn = [z16(ng) for _ in range(num_slots)]
        self.vst = [z16(ng) for _ in range(num_slots)]
        self.tail_k = [z16(group) for _ in range(num_slots)]
        self.tail_v = [z16(group) for _ in range(num_slots)]
        self.pos = self.first = self.written = self.qlen = self.pg = 0
        self.staging = None
        self.staging_pos = 0

    # ---- prefill (kvattn.py:647-666, 745-783)

    def begin_prefill(self, total_len: int) -> None:
        if total_len <= 0 or total_len > self.max_len:
            raise ValueError(f"prefill length {total_len} outside (0, {self.max_len}]")
        self.staging = [(np.zeros((self.h, total_len, self.d), np.float16),
                         np.zeros((self.h, total_len, self.d), np.float16))
                        for _ in range(self.num_slots)]

    def set_prefill_pos(self, off: int) -> None:
        self.pos = int(off)
        self.staging_pos = int(off)

    def finish_prefill(self, total: int) -> None:
        """Quantize whole groups of the staging area, fill the ring with the newest
        <=64 tokens, set the scalars and drop the staging area (``kvattn.py:745-783``)."""
        g = self.group
        q = total // g * g
        ng = q // g
        for layer in range(self.num_slots):
            sk, sv = self.staging[layer]
            if ng:
                kq, kmn, kst = okq.quantize_int8_token(sk[:, :q], g)
                vq, vmn, vst = okq.quantize_int8_token(sv[:, :q], g)
                self.kq[layer][:, :q] = kq
                self.vq[layer][:, :q] = vq
                self.kmn[layer][:, :ng] = kmn
                self.kst[layer][:, :ng] = kst
                self.vmn[layer][:, :ng] = vmn
                self.vst[layer][:, :ng] = vst
            take = min(total, g)
            if take:
                slots = np.arange(total - take, total) % g
                self.tail_k[layer][:, slots] = sk[:, total - take:total]
                self.tail_v[layer][:, slots] = sv[:, total - take:total]
        self.pos, self.first, self.written, self.qlen, self.pg = total, 0, total, q, ng
        self.staging = None

    # ---- decode append (kvattn.py:668-743)

    def update(self, key, value, layer: int) -> None:
        """``key``/``value`` [Hkv, n, D] fp16."""
        if self.staging is not None:
            n = key.shape[1]
            sk, sv = self.staging[layer]
            start = self.staging_pos
            sk[:, start:start + n] = key
            sv[:, start:start + n] = value
            return
        if key.shape[1] != 1:
            raise RuntimeError("without a staging area only one decode token can be appended")
        slot = self.pos % self.group
        self.tail_k[layer][:, slot] = key[:, 0]
        self.tail_v[layer][:, slot] = value[:, 0]
        self._quantize_ring(layer, self.pos // self.group)
        self._sync_scalars()

    def _quantize_ring(self, layer: int, g: int) -> None:
        """Quantize all 64 ring slots, in slot order, into group ``g`` (``kvattn.py:716-743``)."""
        lo = g * self.group
        for tail, codes, mn, st in ((self.tail_k, self.kq, self.kmn, self.kst),
                                    (self.tail_v, self.vq, self.vmn, self.vst)):
            q, m, s = okq.quantize_int8_token(tail[layer], self.group)
            codes[layer][:, lo:lo + self.group] = q
            mn[layer][:, g] = m[:, 0]
            st[layer][:, g] = s[:, 0]

    def _sync_scalars(self) -> None:
        """``_written = pos + 1``, ``_qlen = 64 * floor(_written / 64)``, ``_pg = _qlen / 64``
        (``kvattn.py:699-710``)."""
        self.written = self.pos + 1
        self.qlen = self.written // self.group * self.group
        self.pg = self.qlen // self.group

    # ---- attention (kvattn.py:819-862)

    def ring_mask(self) -> np.ndarray:
        """Slot ``i`` holds absolute position ``p = u - ((u - i) mod 64)``, ``u = _written - 1``;
        it is valid iff ``_qlen <= p <= u`` and ``p >= first``."""
        u = self.written - 1
        i = np.arange(self.group)
        p = u - np.mod(u - i, self.group)
        return (p >= self.qlen) & (p <= u) & (p >= self.first)

    def attend_exact(self, q, layer: int) -> np.ndarray:
        """One softmax over (dequantized prefix) U (valid ring slots), in fp64, rounded to fp16.

        This is the value both the reference's two-part merge and a fused kernel approximate.
        """
        n_g = self.pg
        qlen = self.qlen
        k16 = okq.dequantize_int8_token(self.kq[layer][:, :qlen], self.kmn[layer][:, :n_g],
                                        self.kst[layer][:, :n_g], self.group)
        v16 = okq.dequantize_int8_token(self.vq[layer][:, :qlen], self.vmn[layer][:, :n_g],
                                        self.vst[layer][:, :n_g], self.group)
        mask = self.ring_mask()
        k_all = np.concatenate([k16, self.tail_k[layer][:, mask]], axis=1)
        v_all = np.concatenate([v16, self.tail_v[layer][:, mask]], axis=1)
        out, _ = oattn.attend_fp16_kv(q, k_all, v_all)
        return out.astype(np.float16)

    def attend_two_part(self, q, layer: int) -> np.ndarray:
        """The reference's structure: fp16 prefix output and lse, fp16 tail output and lse,
        log-sum-exp merge rounded to fp16 (``kvattn.py:842-862``)."""
        out_p, lse_p = oattn.int8_attn_decode(q, self.kq[layer], self.kmn[layer], self.kst[layer],
                                              self.vq[layer], self.vmn[layer], self.vst[layer],
                                              self.qlen, self.group)
        out_t, lse_t = oattn.tail_attend(q, self.tail_k[layer], self.tail_v[layer], self.ring_mask())
        return oattn.lse_merge(out_p, lse_p, out_t, lse_t)

    def nbytes(self) -> int:
        """Resident bytes: codes + rulers + ring (``kvattn.py:866-872``)."""
        per_layer = (2 * self.kq[0].nbytes + 4 * self.kmn[0].nbytes + 2 * self.tail_k[0].nbytes)
        return per_layer * self.num_slots


def decode_trajectory(k, v, qs, n0: int, group: int = 64, scale: float | None = None) -> np.ndarray:
    """Outputs of every decode step of a streaming cache, computed in batches (checker only).

    A prefill of ``n0`` tokens is followed by ``S = len(qs)`` decode steps: step i appends token
    ``p = n0 + i`` of ``k`` / ``v`` (``[Hkv, n0 + S, D]`` fp16) and attends with ``qs[i]``
    (``[Hq, D]`` fp16). Each step's value is what :meth:`StreamCache.attend_exact` computes after
    that append: one softmax (fp64) over the int8 prefix ``[0, qlen)``, ``qlen = 64 floor((p + 1)
    / 64)``, dequantized, and the fp16 ring tokens ``[qlen, p]``. An int8 group is the quantizer's
    rounding of its 64 fp16 tokens (the prefill quantizes whole groups; a decode group is the ring
    requantized when its 64th token lands, ``kvattn.py:716-743``), so the prefix is dequantized
    once. Steps that share ``qlen`` share their keys and are computed together, the ring tokens
    under a causal mask. Returns fp64 ``[S, Hq, D]``.
    """
    k = np.asarray(k)
    v = np.asarray(v)
    qs = np.asarray(qs)
    hkv, _, d = k.shape
    S, hq, _ = qs.shape
    gq = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    total = n0 + S
    full = total // group * group
    deq_k = okq.dequantize_int8_token(*okq.quantize_int8_token(k[:, :full], group), group).astype(np.float64)
    deq_v = okq.dequantize_int8_token(*okq.quantize_int8_token(v[:, :full], group), group).astype(np.float64)
    kf, vf = k.astype(np.float64), v.astype(np.float64)
    out = np.zeros((S, hq, d))
    p_all = n0 + np.arange(S)
    qlen_all = (p_all + 1) // group * group
    for qlen in np.unique(qlen_all):
        idx = np.nonzero(qlen_all == qlen)[0]
        ps = p_all[idx]
        t_end = int(ps.max()) + 1  # ring tokens [qlen, t_end)
        ring_pos = np.arange(qlen, t_end)
        keep = ring_pos[None, :] <= ps[:, None]  # [steps, ring tokens]
        for h in range(hkv):
            kk = np.concatenate([deq_k[h, :qlen], kf[h, qlen:t_end]], 0)
            vv = np.concatenate([deq_v[h, :qlen], vf[h, qlen:t_end]], 0)
            q = qs[idx, h * gq:(h + 1) * gq].astype(np.float64)  # [steps, gq, D]
            s = (q @ kk.T) * scale  # [steps, gq, keys]
            s[:, :, qlen:][~np.broadcast_to(keep[:, None, :], s[:, :, qlen:].shape)] = -np.inf
            s -= s.max(axis=2, keepdims=True)
            w = np.exp(s)
            out[idx, h * gq:(h + 1) * gq] = (w @ vv) / w.sum(axis=2, keepdims=True)
    return out
