"""numpy restatement of the reference's int8 KV quantizers (checker only).

Every array operation here is IEEE fp32 (numpy performs no FMA contraction and
``np.rint`` rounds half to even, as ``torch.round`` does), so the outputs are
bit-identical to the reference's torch-on-CPU arithmetic.
"""

from __future__ import annotations

import numpy as np

BYTE_MAX = np.float32(255.0)
STEP_FLOOR = np.float32(1e-8)  # `clamp_min(1e-8)` on an fp32 tensor: the literal is rounded to fp32
SYM_MAX = np.float32(127.0)


def _f32(x) -> np.ndarray:
    return np.asarray(x).astype(np.float32)


def quantize_int8_token(x, group_size: int):
    """Token-axis asymmetric int8, one (min, step) ruler per channel per group of tokens.

    Restates ``src/nova/kvquant.py:136-149``: pad the token axis to a multiple
    of ``group_size`` by repeating the last token, take fp32 min/max over each
    group, ``step = max((max - min) / 255, 1e-8)``, codes
    ``clamp(rint((x - min) / step), 0, 255)``; mins and steps stored as fp16.
    ``x``: ``[..., n, dim]`` -> ``(uint8 [..., n, dim], fp16 [..., ceil(n/gs), dim] x2)``.
    """
    xf = _f32(x)
    *lead, n, dim = xf.shape
    gs = int(group_size or n)
    pad = (-n) % gs
    if pad:
        idx = np.minimum(np.arange(n + pad), n - 1)
        xf = np.take(xf, idx, axis=-2)
    g = xf.reshape(*lead, (n + pad) // gs, gs, dim)
    xmin = g.min(axis=-2)
    xmax = g.max(axis=-2)
    step = np.maximum((xmax - xmin) / BYTE_MAX, STEP_FLOOR)
    q = np.clip(np.rint((g - xmin[..., None, :]) / step[..., None, :]), 0, 255)
    q = q.astype(np.uint8).reshape(*lead, n + pad, dim)[..., :n, :]
    return np.ascontiguousarray(q), xmin.astype(np.float16), step.astype(np.float16)


def dequantize_int8_token(q, mins, steps, group_size: int, dtype=np.float16):
    """Inverse of :func:`quantize_int8_token` (``src/nova/kvquant.py:167-176``).

    ``fp16(fp32(q) * fp32(step16) + fp32(min16))``: the product is exact in fp32,
    the add rounds once to fp32, then once more to fp16.
    """
    q = np.asarray(q)
    *lead, n, dim = q.shape
    gs = int(group_size or n)
    pad = (-n) % gs
    qf = q.astype(np.float32)
    if pad:
        idx = np.minimum(np.arange(n + pad), n - 1)
        qf = np.take(qf, idx, axis=-2)
    g = qf.reshape(*lead, (n + pad) // gs, gs, dim)
    x = g * _f32(steps)[..., None, :] + _f32(mins)[..., None, :]
    return x.reshape(*lead, n + pad, dim)[..., :n, :].astype(dtype)


def quantize_int8_channel(x, group_size: int):
    """Channel-axis asymmetric int8, one ruler per token per group of channels.

    Restates ``src/nova/kvquant.py:128-134``.
    ``x``: ``[..., n, dim]`` -> ``(uint8 [..., n, dim], fp16 [..., n, dim/gs] x2)``.
    """
    xf = _f32(x)
    dim = xf.shape[-1]
    gs = int(group_size or dim)
    if dim % gs:
        raise ValueError(f"head_dim {dim} is not divisible by group_size {gs}")
    g = xf.reshape(*xf.shape[:-1], dim // gs, gs)
    xmin = g.min(axis=-1)
    xmax = g.max(axis=-1)
    step = np.maximum((xmax - xmin) / BYTE_MAX, STEP_FLOOR)
    q = np.clip(np.rint((g - xmin[..., None]) / step[..., None]), 0, 255)
    return q.astype(np.uint8).reshape(xf.shape), xmin.astype(np.float16), step.astype(np.float16)


def dequantize_int8_channel(q, mins, steps, group_size: int, dtype=np.float16):
    """Inverse of :func:`quantize_int8_channel` (``src/nova/kvquant.py:161-165``)."""
    q = np.asarray(q)
    dim = q.shape[-1]
    gs = int(group_size or dim)
    g = q.astype(np.float32).reshape(*q.shape[:-1], dim // gs, gs)
    x = g * _f32(steps)[..., None] + _f32(mins)[..., None]
    return x.reshape(q.shape).astype(dtype)


def quantize_int8(x, group_size: int = 32, axis: str = "channel"):
    """Dispatch mirroring ``quantize_int8(x, group_size, axis)`` (``src/nova/kvquant.py:118-126``)."""
    if axis not in ("channel", "token"):
        raise ValueError(f"axis must be 'channel' or 'token', got {axis!r}")
    if axis == "channel":
        return quantize_int8_channel(x, group_size)
    return quantize_int8_token(x, group_size)


def dequantize_int8(q, mins, steps, group_size: int = 32, axis: str = "channel", dtype=np.float16):
    """Dispatch mirroring ``dequantize_int8`` (``src/nova/kvquant.py:152-176``)."""
    if axis == "channel":
        return dequantize_int8_channel(q, mins, steps, group_size, dtype)
    return dequantize_int8_token(q, mins, steps, group_size, dtype)


# ---------------------------------------------------------------- per-token symmetric ("tok")
# Extension with no counterpart in the reference: one symmetric absmax scale per
# (token, kv_head) row. Rounding conventions follow kvquant: fp32 arithmetic,
# round-half-even, a 1e-8 floor on the fp32 scale, the scale stored as fp16 and
# the codes computed with the fp32 scale.


def quantize_tok(x):
    """``x``: ``[..., n, dim]`` -> ``(int8 codes [..., n, dim], fp16 scale [..., n])``.

    ``scale = max(max|x| / 127, 1e-8)`` in fp32; ``code = clamp(rint(x / scale), -127, 127)``.
    """
    xf = _f32(x)
    amax = np.abs(xf).max(axis=-1)
    scale = np.maximum(amax / SYM_MAX, STEP_FLOOR)
    q = np.clip(np.rint(xf / scale[..., None]), -127, 127).astype(np.int8)
    return q, scale.astype(np.float16)


def dequantize_tok(q, scale, dtype=np.float16):
    """``fp16(fp32(code) * fp32(scale16))`` — the product is exact in fp32."""
    return (np.asarray(q).astype(np.float32) * _f32(scale)[..., None]).astype(dtype)


# ---------------------------------------------------------------- byte accounting


def bytes_per_token_int8(num_slots: int, num_kv_heads: int, head_dim: int, group_k: int = 32,
                         group_v: int = 0, k_axis: str = "channel", token_group: int = 64):
    """int8 branch of ``bytes_per_token`` (``src/nova/kvquant.py:268-279``).

    Restated literally: the metadata per head is ``2 * 2 * (dim // g)`` bytes per
    token, with ``g = token_group`` when K groups run along the token axis.
    """
    def one8(dim: int, group: int) -> float:
        g = dim if group in (0, None) else group
        return dim * 1 + 2 * 2 * (dim // g)

    kv16 = 2 * head_dim * 2
    k8 = one8(head_dim, token_group if k_axis == "token" else group_k)
    v8 = one8(head_dim, group_v)
    return {
        "fp16_kv": kv16 * num_slots * num_kv_heads,
        "int8_kv": (k8 + v8) * num_slots * num_kv_heads,
        "ratio": kv16 / (k8 + v8),
    }
