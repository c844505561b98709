"""int8 KV quantizers on the GPU — drop-in for ``nova.kvquant``'s int8 path.

Same call signatures and outputs as ``quantize_int8`` / ``dequantize_int8``
(src/nova/kvquant.py:118-176), computed by the HIP kernels of ``libnova_kv.so``
and bit-exact with the reference's rounding. Tensors must live on the GPU; there
is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib

GROUP_K = 32  # default group size of the reference (src/nova/kvquant.py:52)
BYTE_MAX = 255

_DT = {torch.float16: _lib.NKV_F16, torch.bfloat16: _lib.NKV_BF16, torch.float32: _lib.NKV_F32}


def _on_gpu(x: torch.Tensor, name: str) -> None:
    if not x.is_cuda:
        raise ValueError(f"{name} must be on the GPU (nova_amd runs the HIP kernels only)")


def _slabs(x: torch.Tensor):
    """View ``[..., n, dim]`` as ``rows`` slabs of a contiguous ``[n, dim]`` block.

    Returns ``(rows, row_stride)`` or None when the layout needs a copy.
    """
    *lead, n, dim = x.shape
    if x.stride(-1) != 1 or (n > 1 and x.stride(-2) != dim):
        return None
    rows = 1
    for s in lead:
        rows *= s
    if rows <= 1:
        return rows, n * dim
    # the leading dims must collapse into one stride
    stride = x.stride(len(lead) - 1)
    expect = stride
    for i in range(len(lead) - 1, -1, -1):
        if lead[i] != 1 and x.stride(i) != expect:
            return None
        expect *= lead[i]
    return rows, stride


def _prep(x: torch.Tensor):
    sl = _slabs(x)
    if sl is None or x.data_ptr() % 16:
        x = x.contiguous()
        sl = _slabs(x)
    return x, sl[0], sl[1]


def quantize_int8(x: torch.Tensor, group_size: int = GROUP_K, axis: str = "channel"):
    """Asymmetric int8 quantization. ``x`` ``[..., n, dim]`` -> ``(uint8, mins, steps)``.

    - ``axis="channel"``: groups of ``group_size`` channels along ``dim``, one ruler per
      token (``src/nova/kvquant.py:128-134``); rulers ``[..., n, dim/gs]``.
    - ``axis="token"``: groups of ``group_size`` tokens (0 = all), one ruler per channel
      per group (``kvquant.py:136-149``); rulers ``[..., ceil(n/gs), dim]``.
    Rulers are fp16; ``step = max((max-min)/255, 1e-8)`` in fp32 and
    ``code = clamp(rint((x-min)/step), 0, 255)``, exactly as the reference.
    """
    if axis not in ("channel", "token"):
        raise ValueError(f"axis must be 'channel' or 'token', got {axis!r}")
    _on_gpu(x, "x")
    if x.dtype not in _DT:
        x = x.float()
    *lead, n, dim = x.shape
    if axis == "channel":
        gs = int(group_size or dim)
        if dim % gs:
            raise ValueError(f"head_dim {dim} 不能被 group_size {gs} 整除")
        sshape = (*lead, n, dim // gs)
    else:
        gs = int(group_size or n)
        sshape = (*lead, -(-n // gs) if n else 0, dim)
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    mins = torch.empty(sshape, dtype=torch.float16, device=x.device)
    steps = torch.empty(sshape, dtype=torch.float16, device=x.device)
    if x.numel() == 0:
        return q, mins, steps
    xc, rows, xrs = _prep(x)
    nsc = sshape[-2] * sshape[-1]
    _lib.call("nkv_quantize_int8", xc.data_ptr(), _DT[xc.dtype], xrs, rows, n, dim, gs,
              _lib.NKV_AXIS_CHANNEL if axis == "channel" else _lib.NKV_AXIS_TOKEN,
              q.data_ptr(), n * dim, mins.data_ptr(), steps.data_ptr(), nsc, _lib.stream_ptr(x.device))
    return q, mins, steps


def quantize_int8_into(x: torch.Tensor, group_size: int, q: torch.Tensor, mins: torch.Tensor,
                       steps: torch.Tensor) -> None:
    """Token-axis quantization written straight into strided cache slices.

    ``x`` ``[1, H, n, D]`` (any slab stride), ``q`` ``[1, H, n, D]`` uint8 slice,
    ``mins``/``steps`` ``[1, H, ceil(n/gs), D]`` fp16 slices — the in-place form of
    ``KVInt8Cache.finish_prefill``'s bulk quantize (src/nova/kvattn.py:761-769).
    """
    _on_gpu(x, "x")
    *lead, n, dim = x.shape
    xc, rows, xrs = _prep(x)
    for t, nm in ((q, "q"), (mins, "mins"), (steps, "steps")):
        if t.stride(-1) != 1 or t.stride(-2) != dim:
            raise ValueError(f"{nm} rows must be contiguous")
    _lib.call("nkv_quantize_int8", xc.data_ptr(), _DT[xc.dtype], xrs, rows, n, dim, int(group_size),
              _lib.NKV_AXIS_TOKEN, q.data_ptr(), q.stride(-3), mins.data_ptr(), steps.data_ptr(),
              mins.stride(-3), _lib.stream_ptr(x.device))


def dequantize_int8(
    q: torch.Tensor,
    mins: torch.Tensor,
    steps: torch.Tensor,
    group_size: int = GROUP_K,
    axis: str = "channel",
    dtype: torch.dtype = torch.float16,
) -> torch.Tensor:
    """Inverse of :func:`quantize_int8` (``src/nova/kvquant.py:152-176``):
    ``dtype(fp32(q) * fp32(step) + fp32(min))``."""
    if axis not in ("channel", "token"):
        raise ValueError(f"axis must be 'channel' or 'token', got {axis!r}")
    _on_gpu(q, "q")
    if dtype not in _DT:
        raise ValueError(f"unsupported output dtype {dtype}")
    *lead, n, dim = q.shape
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    if q.numel() == 0:
        return out
    if axis == "channel":
        gs = int(group_size or dim)
    else:
        gs = int(group_size or n)
    qc = q.contiguous()
    mc = mins.contiguous()
    sc = steps.contiguous()
    if mc.dtype != torch.float16:
        mc = mc.to(torch.float16)
    if sc.dtype != torch.float16:
        sc = sc.to(torch.float16)
    rows = qc.numel() // (n * dim)
    nsc = mc.shape[-2] * mc.shape[-1]
    _lib.call("nkv_dequantize_int8", qc.data_ptr(), n * dim, mc.data_ptr(), sc.data_ptr(), nsc, rows, n, dim,
              gs, _lib.NKV_AXIS_CHANNEL if axis == "channel" else _lib.NKV_AXIS_TOKEN, out.data_ptr(),
              _DT[dtype], n * dim, _lib.stream_ptr(q.device))
    return out


def roundtrip_int8(x: torch.Tensor, group_size: int = GROUP_K, axis: str = "channel",
                   dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Quantize then dequantize (``src/nova/kvquant.py:179-186``)."""
    q, mins, steps = quantize_int8(x, group_size, axis)
    return dequantize_int8(q, mins, steps, group_size, axis, dtype)


def bytes_per_token(num_slots: int, num_kv_heads: int, head_dim: int, group_k: int = GROUP_K,
                    group_v: int = 0, bits: int = 8, k_axis: str = "channel", token_group: int = 64):
    """KV bytes per token, fp16 vs int8 with rulers — the int8 branch of the reference's
    accounting (``src/nova/kvquant.py:232-289``)."""
    if int(bits) != 8:
        raise NotImplementedError("only the int8 accounting is part of this path")

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
