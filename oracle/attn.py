"""numpy restatement of the decode attention the int8 path must reproduce (checker only)."""

from __future__ import annotations

import numpy as np

from . import kvquant as okq

LN2 = float(np.log(2.0))


def _softmax_attend(qg: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float):
    """One KV head: ``qg`` [gq, D], ``k``/``v`` [n, D] (any float dtype) -> (out [gq, D], lse [gq]) in fp64."""
    qg = qg.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    if k.shape[0] == 0:
        return np.zeros((qg.shape[0], v.shape[1])), np.full(qg.shape[0], -np.inf)
    s = (qg @ k.T) * scale
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(axis=1, keepdims=True)
    return (p @ v) / l, (m + np.log(l))[:, 0]


def attend_fp16_kv(q, k16, v16, scale=None):
    """Decode-step attention over fp16 K/V with GQA head sharing, in fp64.

    ``q`` [Hq, D]; ``k16``/``v16`` [Hkv, n, D]. Q head ``h`` reads KV head
    ``h // (Hq // Hkv)`` (the ``repeat_kv`` expansion of ``tests/test_kvattn.py:67-68``).
    Returns ``(out fp64 [Hq, D], lse fp64 [Hq])``.
    """
    q = np.asarray(q)
    hq, d = q.shape
    hkv = k16.shape[0]
    gq = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    out = np.zeros((hq, d))
    lse = np.zeros(hq)
    for h in range(hkv):
        o, ls = _softmax_attend(q[h * gq:(h + 1) * gq], k16[h], v16[h], scale)
        out[h * gq:(h + 1) * gq] = o
        lse[h * gq:(h + 1) * gq] = ls
    return out, lse


def int8_attn_decode(q, kq, kmn, kst, vq, vmn, vst, used: int, group: int = 64):
    """Reference numerics of the fused int8 decode kernel: dequantize ``[0, used)``
    with the stored fp16 rulers, then softmax attention (``tests/test_kvattn.py:62-70``).

    ``q`` [Hq, D] fp16; ``kq``/``vq`` [Hkv, L, D] uint8; rulers [Hkv, ceil(L/group), D] fp16.
    Returns ``(out fp16 [Hq, D], lse fp32 [Hq])``; ``used == 0`` gives zeros and -inf
    (``src/nova/kvattn.py:387-391``).
    """
    hq, d = np.asarray(q).shape
    if used == 0:
        return np.zeros((hq, d), np.float16), np.full(hq, -np.inf, np.float32)
    n_g = -(-used // group)
    k16 = okq.dequantize_int8_token(kq[:, :used], kmn[:, :n_g], kst[:, :n_g], group)
    v16 = okq.dequantize_int8_token(vq[:, :used], vmn[:, :n_g], vst[:, :n_g], group)
    out, lse = attend_fp16_kv(q, k16, v16)
    return out.astype(np.float16), lse.astype(np.float32)


def tail_attend(q, k, v, mask):
    """fp16 ring attention and its log-sum-exp (``src/nova/kvattn.py:447-482``).

    ``q`` [Hq, D]; ``k``/``v`` [Hkv, R, D] fp16; ``mask`` bool [R]. An empty mask
    gives out 0 and lse -inf (``kvattn.py:476-481``).
    """
    mask = np.asarray(mask, bool)
    hq, d = np.asarray(q).shape
    if not mask.any():
        return np.zeros((hq, d), np.float16), np.full(hq, -np.inf, np.float32)
    out, lse = attend_fp16_kv(q, k[:, mask], v[:, mask])
    return out.astype(np.float16), lse.astype(np.float32)


def lse_merge(out_p, lse_p, out_t, lse_t):
    """Merge two attention partials by their log-sum-exp (``src/nova/kvattn.py:852-862``).

    ``out = (o_p e^{lse_p} + o_t e^{lse_t}) / (e^{lse_p} + e^{lse_t})`` with the
    max subtracted, per head; the result is rounded to fp16.
    """
    lp = np.asarray(lse_p, np.float64)[:, None]
    lt = np.asarray(lse_t, np.float64)[:, None]
    m = np.maximum(lp, lt)
    wp = np.exp(lp - m)
    wt = np.exp(lt - m)
    merged = (np.asarray(out_p, np.float64) * wp + np.asarray(out_t, np.float64) * wt) / (wp + wt)
    return merged.astype(np.float16)


# ---------------------------------------------------------------- per-token symmetric ("tok")


def tok_attn_decode(q, kq, ks, vq, vs, used: int):
    """Decode attention over the per-token symmetric int8 cache (extension, no reference
    counterpart): dequantize ``fp16(code * scale16)`` then softmax attention.

    ``kq``/``vq`` [Hkv, L, D] int8; ``ks``/``vs`` [Hkv, L] fp16.
    """
    hq, d = np.asarray(q).shape
    if used == 0:
        return np.zeros((hq, d), np.float16), np.full(hq, -np.inf, np.float32)
    k16 = okq.dequantize_tok(kq[:, :used], ks[:, :used])
    v16 = okq.dequantize_tok(vq[:, :used], vs[:, :used])
    out, lse = attend_fp16_kv(q, k16, v16)
    return out.astype(np.float16), lse.astype(np.float32)


# ---------------------------------------------------------------- chunked prefill


def chunk_prefill_attend(q, kq, kmn, kst, vq, vmn, vst, used: int, k_chunk, v_chunk, heads=None):
    """Causal attention of a prefill chunk over the int8t64 cache, an fp16 history and itself.

    ``q`` [Hq, M, D] fp16; ``kq``/``vq`` [Hkv, L, D] uint8 with rulers [Hkv, ceil(L/64), D]
    (``used`` a multiple of 64); ``k_chunk``/``v_chunk`` [Hkv, m, D] fp16 with ``m >= M``: the
    first ``m - M`` tokens are an fp16 history at positions ``used ..``, the last ``M`` the
    chunk, so query token i sits at position ``used + m - M + i``. Token i attends to the cache
    tokens [0, used), dequantized as ``dequantize_int8_token`` does, to the history and to chunk
    tokens [0, i] — the reference's ``attend_prefill`` (``src/nova/kvattn.py:791-815``: causal
    SDPA over the staged fp16 positions before and including each query) with the part already
    quantized read from int8. Returns fp64 ``[Hq, M, D]`` (only the KV heads in ``heads`` when
    given; other rows are 0).
    """
    q = np.asarray(q)
    hq, n, d = q.shape
    hkv, m = k_chunk.shape[0], k_chunk.shape[1]
    assert m >= n, "the fp16 K/V must hold at least the chunk"
    gq = hq // hkv
    n_g = used // 64
    out = np.zeros((hq, n, d))
    for h in (range(hkv) if heads is None else heads):
        if used:
            kc = okq.dequantize_int8_token(kq[h:h + 1, :used], kmn[h:h + 1, :n_g], kst[h:h + 1, :n_g], 64)[0]
            vc = okq.dequantize_int8_token(vq[h:h + 1, :used], vmn[h:h + 1, :n_g], vst[h:h + 1, :n_g], 64)[0]
            k = np.concatenate([kc, k_chunk[h]], 0).astype(np.float64)
            v = np.concatenate([vc, v_chunk[h]], 0).astype(np.float64)
        else:
            k = k_chunk[h].astype(np.float64)
            v = v_chunk[h].astype(np.float64)
        keypos = np.arange(used + m)
        mask = keypos[None, :] > (used + m - n + np.arange(n))[:, None]  # [M, used + m]
        for j in range(gq):
            s = (q[h * gq + j].astype(np.float64) @ k.T) * d ** -0.5
            s[mask] = -np.inf
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[h * gq + j] = (p @ v) / p.sum(axis=1, keepdims=True)
    return out
