"""int8 KV decode attention and the streaming int8 cache on MI355X — drop-in for ``nova.kvattn``.

Public surface and error behaviour follow src/nova/kvattn.py: ``GROUP_T``, ``CHUNK``,
``PAD_M``, ``int8_attn_decode``, ``pack_int8_kv``, ``tail_attend`` and ``KVInt8Cache``.
Every computation runs in the HIP kernels of ``libnova_kv.so``: decode attention is two
launches (the split-K prefix kernel, then the tail kernel with the ring and the combine),
and the fused ``KVInt8Cache.update_attend`` runs the append inside the first of them. ValueError messages
keep the reference's key terms (解码一步, chunk, group, used, 尺子) so callers that
match on them keep working.

Numerics: codes and rulers are bit-exact with ``kvquant.quantize_int8(x, 64, "token")``;
attention outputs match "dequantize, then softmax attention in fp32" to within the
reference's criterion (<= 2 fp16 ULP or <= 1e-5 absolute for the int8 prefix; the
ring tail is folded into the same softmax instead of a separate fp16 SDPA + log-sum-exp
merge, which only removes two fp16 roundings).
"""

from __future__ import annotations

from typing import Any

import torch
import torch.nn.functional as F

from . import _lib
from .kvquant import quantize_int8, quantize_int8_into

GROUP_T = 64  # tokens per ruler (int8t64), src/nova/kvattn.py:103
CHUNK = 512   # reference split granularity; sizes the caller-visible scratch
PAD_M = 16    # query heads per KV head are padded to 16 MFMA rows

D_SUPPORTED = 128


def _check(x: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    """``src/nova/kvattn.py:256-262``."""
    if not x.is_cuda:
        raise ValueError(f"{name} 必须在 CUDA 上 (must be on the GPU)")
    if x.dtype != dtype:
        raise ValueError(f"{name} 必须是 {dtype}，收到 {x.dtype}")
    if not x.is_contiguous():
        raise ValueError(f"{name} 必须连续 (must be contiguous)")


def _is_capturing() -> bool:
    try:
        return torch.cuda.is_current_stream_capturing()
    except Exception:  # noqa: BLE001
        return False


def _pick_parts(hkv: int, hq: int, groups: int, ws_bytes: int | None, fused: bool = False) -> int:
    """Default prefix parts, capped by what ``ws_bytes`` holds: one partial per KV head per part,
    plus, for the fused decode step, the completion counters."""
    lib = _lib.load()
    parts = int(lib.nkv_attn_default_parts(hkv, groups))
    if ws_bytes is not None:
        per_part = int(lib.nkv_attn_workspace_bytes(hkv, hq, 2)) - int(lib.nkv_attn_workspace_bytes(hkv, hq, 1))
        extra = int(lib.nkv_attn_workspace_bytes(hkv, hq, 1)) - per_part if fused else 0
        fit = (ws_bytes - extra) // per_part
        if fit < 1:
            raise ValueError(f"scratch too small: {ws_bytes} bytes")
        parts = max(1, min(parts, fit))
    return parts


def int8_attn_decode(
    q: torch.Tensor,
    kq: torch.Tensor,
    kmn: torch.Tensor,
    kst: torch.Tensor,
    vq: torch.Tensor,
    vmn: torch.Tensor,
    vst: torch.Tensor,
    *,
    used: int | None = None,
    group: int = GROUP_T,
    chunk: int = CHUNK,
    num_warps: int = 8,
    num_stages: int = 2,
    scratch: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    out: torch.Tensor | None = None,
    lse_out: torch.Tensor | None = None,
    prefix_groups: int | torch.Tensor = -1,
    used_t: torch.Tensor | None = None,
    prefix_groups_t: torch.Tensor | None = None,
    n_splits: int | None = None,
) -> torch.Tensor:
    """Fused int8 attention for one decode step (``src/nova/kvattn.py:281-427``).

    - ``q``: fp16 ``[1, H_q, 1, D]`` (RoPE applied)
    - ``kq``/``vq``: uint8 ``[1, H_kv, L, D]``; ``kmn``/``kst``/``vmn``/``vst``: fp16
      ``[1, H_kv, ceil(L/group), D]``
    - ``used``: valid KV length (default ``L``); only ``[0, used)`` is read
    - ``scratch`` ``(pm, pl, pa)`` / ``out`` / ``lse_out``: preallocated buffers (required
      under graph capture); the kernel uses ``pa``'s memory as its partial workspace
    - ``prefix_groups``: number of valid rulers (-1 = all of ``ceil(used/group)``)
    - ``used_t`` / ``prefix_groups_t``: device int64 ``[1]`` scalars read inside the
      kernel (graph-safe); they override ``used`` / ``prefix_groups``
    - ``n_splits``: fixes the scratch shape; ``num_warps`` / ``num_stages`` are accepted
      for signature compatibility (the HIP kernel's launch shape is its own)

    Returns fp16 ``[1, H_q, 1, D]``.
    """
    _lib.load()
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError(f"本核只处理解码一步 (one decode step: q is [1, H_q, 1, D])，收到 {tuple(q.shape)}")
    if q.shape[0] != 1:
        raise ValueError("batch 必须为 1")
    _check(q, "q", torch.float16)
    for name, t, dt in (("kq", kq, torch.uint8), ("vq", vq, torch.uint8),
                        ("kmn", kmn, torch.float16), ("kst", kst, torch.float16),
                        ("vmn", vmn, torch.float16), ("vst", vst, torch.float16)):
        _check(t, name, dt)

    _, hq, _, d = q.shape
    h_kv, length = kq.shape[1], kq.shape[2]
    if kq.shape != vq.shape:
        raise ValueError(f"kq {tuple(kq.shape)} 与 vq {tuple(vq.shape)} 形状不一致")
    if kmn.shape != kst.shape or kmn.shape != vmn.shape or kmn.shape != vst.shape:
        raise ValueError("四张尺子的形状必须一致 (the four rulers must have one shape)")
    if kmn.shape[0] != 1 or kmn.shape[1] != h_kv or kmn.shape[3] != d:
        raise ValueError(f"尺子形状 {tuple(kmn.shape)} 与 KV {tuple(kq.shape)} 不符")
    if hq % h_kv:
        raise ValueError(f"Q 头 {hq} 不能被 KV 头 {h_kv} 整除")
    gq = hq // h_kv
    if gq > PAD_M:
        raise ValueError(f"每个 KV 头摊到 {gq} 个 Q 头，超过补零上限 {PAD_M}")
    if d & (d - 1):
        raise ValueError(f"head_dim {d} 必须是 2 的幂")
    if group & (group - 1):
        raise ValueError(f"group {group} 必须是 2 的幂")
    if chunk % group:
        raise ValueError(f"chunk {chunk} 必须是 group {group} 的整数倍")
    if kmn.shape[2] != -(-length // group):
        raise ValueError(f"尺子组数 {kmn.shape[2]} != ceil(L/group) = {-(-length // group)}")

    used = length if used is None else int(used)
    if not 0 <= used <= length:
        raise ValueError(f"used={used} 超出 [0, {length}]")
    if not isinstance(prefix_groups, torch.Tensor):
        prefix_groups = int(prefix_groups)
        if prefix_groups < 0:
            prefix_groups = -(-used // group)
        elif prefix_groups > kmn.shape[2]:
            raise ValueError(f"prefix_groups={prefix_groups} 超过尺子组数 {kmn.shape[2]}")
    elif used_t is None:
        prefix_groups = int(prefix_groups.item())  # eager host value, as the reference's fill_
    else:
        prefix_groups_t = prefix_groups if prefix_groups_t is None else prefix_groups_t
        prefix_groups = -1

    used_is_device = used_t is not None
    if used_is_device:
        if tuple(used_t.shape) != (1,) or used_t.dtype != torch.int64 or not used_t.is_cuda:
            raise ValueError(f"used_t 必须是 CUDA int64 [1]，收到 {tuple(used_t.shape)} {used_t.dtype}")
        t = prefix_groups_t
        if t is None or tuple(t.shape) != (1,) or t.dtype != torch.int64 or not t.is_cuda:
            raise ValueError("prefix_groups_t 必须是 CUDA int64 [1]")
    if out is None:
        out = torch.empty((1, hq, 1, d), dtype=torch.float16, device=q.device)
    elif out.shape != (1, hq, 1, d) or out.dtype != torch.float16 or not out.is_cuda:
        raise ValueError(f"out 形状/类型不对：{tuple(out.shape)} {out.dtype}")
    if lse_out is not None and (
        tuple(lse_out.shape) != (1, hq) or lse_out.dtype != torch.float32 or not lse_out.is_cuda
    ):
        raise ValueError(f"lse_out 形状/类型不对：{tuple(lse_out.shape)} {lse_out.dtype}")

    n_splits = -(-used // chunk) if n_splits is None else int(n_splits)
    if used_is_device or used:
        if n_splits < 1:
            raise ValueError(f"n_splits={n_splits} 必须 ≥ 1")
    ws_given = None
    if scratch is not None:
        pm, pl, pa = scratch
        want = (h_kv, n_splits, PAD_M)
        if tuple(pm.shape) != want or tuple(pl.shape) != want or tuple(pa.shape) != (*want, d):
            raise ValueError(f"scratch 形状不对：要 {want} / {(*want, d)}，"
                             f"收到 {tuple(pm.shape)} / {tuple(pa.shape)}")
        ws_given = pa
    if group != GROUP_T or d != D_SUPPORTED:
        raise NotImplementedError(f"the HIP kernel reads 64-token rulers and head_dim 128 (group={group}, D={d})")

    groups = kmn.shape[2] if used_is_device else -(-min(used, prefix_groups * group) // group)
    if ws_given is not None:
        n_parts = _pick_parts(h_kv, hq, groups, ws_given.numel() * 4)
        ws = ws_given
        ws_bytes = ws_given.numel() * 4
    else:
        n_parts = _pick_parts(h_kv, hq, groups, None)
        ws_bytes = int(_lib.load().nkv_attn_workspace_bytes(h_kv, hq, n_parts))
        cached = _lib._WORKSPACES.get(f"{q.device}/decode")
        if _is_capturing() and (cached is None or cached.numel() < ws_bytes):
            raise ValueError("under graph capture pass scratch=(pm, pl, pa) (no workspace is allocated there)")
        ws = _lib.workspace(q.device, ws_bytes, "decode")
        ws_bytes = ws.numel()
    _lib.call(
        "nkv_attn_decode_t64", q.data_ptr(), kq.data_ptr(), kmn.data_ptr(), kst.data_ptr(), vq.data_ptr(),
        vmn.data_ptr(), vst.data_ptr(), hq, h_kv, d, length, used, prefix_groups,
        _lib.ptr(used_t), _lib.ptr(prefix_groups_t), None, None, None, None,
        out.data_ptr(), _lib.ptr(lse_out), ws.data_ptr(), ws_bytes, n_parts,
        _lib.stream_ptr(q.device))
    return out


def int8_prefill_attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kq: torch.Tensor,
                        kmn: torch.Tensor, kst: torch.Tensor, vq: torch.Tensor, vmn: torch.Tensor,
                        vst: torch.Tensor, used: int, out: torch.Tensor | None = None,
                        scratch: torch.Tensor | None = None, splits: int = 0) -> torch.Tensor:
    """Causal attention of a prefill chunk over an int8t64 cache and itself (MFMA kernels).

    The chunk's ``query`` ``[1, Hq, n, 128]`` (positions ``used .. used + n - 1``) attends to
    the cache's first ``used`` tokens (a multiple of 64: ``kq``/``vq`` ``[1, Hkv, L, 128]``
    uint8, rulers ``[1, Hkv, ceil(L/64), 128]``) and causally to its own fp16 ``key`` /
    ``value`` ``[1, Hkv, n, 128]``. It computes what ``KVInt8Cache.attend_prefill`` does
    over fp16 staging (src/nova/kvattn.py:791-815) with the cached part read as int8.
    Returns ``out`` ``[1, Hq, n, 128]`` fp16.
    """
    for t, nm in ((query, "query"), (key, "key"), (value, "value")):
        _check(t, nm, torch.float16)
    for t, nm in ((kq, "kq"), (vq, "vq")):
        _check(t, nm, torch.uint8)
    for t, nm in ((kmn, "kmn"), (kst, "kst"), (vmn, "vmn"), (vst, "vst")):
        _check(t, nm, torch.float16)
    _, hq, n, d = query.shape
    _, hkv, cap, _ = kq.shape
    if key.shape != (1, hkv, n, d) or value.shape != key.shape:
        raise ValueError(f"key / value must be [1, {hkv}, {n}, {d}]")
    if used % GROUP_T or not 0 <= used <= cap:
        raise ValueError(f"used={used} must be a multiple of {GROUP_T} in [0, {cap}]")
    if out is None:
        out = torch.empty_like(query)
    lib = _lib.load()
    if splits <= 0:
        splits = int(lib.nkv_prefill_default_splits(hkv, hq, n, used))
    need = int(lib.nkv_prefill_workspace_bytes(hkv, hq, n, splits))
    if scratch is None or scratch.numel() * scratch.element_size() < need:
        scratch = _lib.workspace(query.device, need)
    _lib.call("nkv_prefill_attn_t64", query.data_ptr(), key.data_ptr(), value.data_ptr(), n, kq.data_ptr(),
              kmn.data_ptr(), kst.data_ptr(), vq.data_ptr(), vmn.data_ptr(), vst.data_ptr(), cap, used, hq, hkv,
              d, out.data_ptr(), scratch.data_ptr(), scratch.numel() * scratch.element_size(), splits,
              _lib.stream_ptr(query.device))
    return out


def pack_int8_kv(k: torch.Tensor, v: torch.Tensor, group: int = GROUP_T):
    """fp16 K/V -> ``(kq, kmn, kst, vq, vmn, vst)`` with the token-axis quantizer
    (``src/nova/kvattn.py:430-441``)."""
    kq, kmn, kst = quantize_int8(k, group, "token")
    vq, vmn, vst = quantize_int8(v, group, "token")
    return (kq.contiguous(), kmn.contiguous(), kst.contiguous(),
            vq.contiguous(), vmn.contiguous(), vst.contiguous())


def tail_attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tail_mask: torch.Tensor):
    """Attention over the fp16 ring and its log-sum-exp (``src/nova/kvattn.py:447-482``).

    - ``q`` fp16 ``[1, H_q, 1, D]``; ``k``/``v`` fp16 ``[1, H_kv, R, D]`` (R <= 64)
    - ``tail_mask`` bool ``[1, 1, 1, R]``, True = slot valid
    Returns ``(out fp16 [1, H_q, 1, D], lse fp32 [1, H_q])``; an empty mask gives out 0
    and lse -inf.
    """
    hq, h_kv = q.shape[1], k.shape[1]
    if hq % h_kv:
        raise ValueError(f"Q 头 {hq} 不能被 KV 头 {h_kv} 整除")
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    _check(qc, "q", torch.float16)
    _check(kc, "k", torch.float16)
    _check(vc, "v", torch.float16)
    slots, d = k.shape[2], k.shape[3]
    mask = tail_mask.reshape(-1)
    if mask.numel() != slots:
        raise ValueError(f"tail_mask has {mask.numel()} entries for {slots} slots")
    mask = mask.to(torch.uint8) if mask.dtype != torch.uint8 else mask.contiguous()
    out = torch.empty((1, hq, 1, d), dtype=torch.float16, device=q.device)
    lse = torch.empty((1, hq), dtype=torch.float32, device=q.device)
    _lib.call("nkv_tail_attend", qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), mask.data_ptr(),
              hq, h_kv, d, slots, out.data_ptr(), lse.data_ptr(), _lib.stream_ptr(q.device))
    return out, lse


class KVInt8Cache:
    r"""Streaming int8 KV cache (``src/nova/kvattn.py:488-880``).

    Resident state per layer: an int8 prefix of whole 64-token groups with fp16
    rulers, and a 64-slot fp16 ring holding the newest tokens (slot = position mod 64).
    Lengths live in device scalars (``pos``, ``first``, ``_written``, ``_qlen``, ``_pg``)
    so a captured decode graph stays valid as the prefix grows.

    Decode step of one layer (graph-safe, no host sync):
    1. ``update()``: one HIP launch writes K/V into ring slot ``pos % 64``, requantizes
       the whole ring into ruler group ``pos // 64`` and sets ``_written = pos + 1``,
       ``_qlen = 64 * floor(_written / 64)``, ``_pg = _qlen / 64``;
    2. ``attend()``: two HIP launches (split-K partials, then ring + combine) attend over
       the int8 prefix ``[0, _qlen)`` and the valid ring slots in a single softmax.
    ``update_attend()`` does both in those two launches, the append running inside the
    first (what the decode loop uses).

    Prefill goes through an fp16 staging area sized to the prompt (``begin_prefill``),
    then ``finish_prefill`` quantizes whole groups with the bulk HIP quantizer, fills the
    ring and frees the staging area.

    Streamed prefill (``begin_prefill(total, stream_chunk=c)``, ``c`` a multiple of 64) keeps
    only the current chunk in fp16: each chunk starts on a group boundary, ``update``
    quantizes its whole groups straight into the int8 cache and writes its newest tokens to
    the ring, and ``attend_prefill`` attends the int8 history plus the fp16 chunk on MFMA
    (the 64-multiple chunking of ``reports/kv-int8-streaming-cache.md:126-131``). Every
    group is quantized from the same 64 fp16 tokens as in the staged path, so the final
    cache state is identical; only the chunk attention reads the history as int8.
    """

    def __init__(
        self,
        num_slots: int,
        num_kv_heads: int,
        head_dim: int,
        max_len: int,
        num_q_heads: int,
        batch: int = 1,
        dtype: torch.dtype = torch.float16,
        device: str | torch.device = "cuda",
        group: int = GROUP_T,
        chunk: int = CHUNK,
        num_warps: int = 8,
        num_stages: int = 2,
    ) -> None:
        if head_dim & (head_dim - 1):
            raise ValueError(f"head_dim {head_dim} 必须是 2 的幂")
        if num_q_heads % num_kv_heads:
            raise ValueError(f"Q 头 {num_q_heads} 不能被 KV 头 {num_kv_heads} 整除")
        if num_q_heads // num_kv_heads > PAD_M:
            raise ValueError(f"每个 KV 头摊到 {num_q_heads // num_kv_heads} 个 Q 头，超过补零上限 {PAD_M}")
        if group & (group - 1):
            raise ValueError(f"group {group} 必须是 2 的幂")
        if chunk % group:
            raise ValueError(f"chunk {chunk} 必须是 group {group} 的整数倍")
        if batch != 1:
            raise ValueError("batch 必须为 1")
        if group != GROUP_T or head_dim != D_SUPPORTED or dtype != torch.float16:
            raise NotImplementedError("the HIP path stores fp16 K/V with 64-token rulers and head_dim 128")
        _lib.load()

        self.num_slots = int(num_slots)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.max_len = int(max_len)
        self.num_q_heads = int(num_q_heads)
        self.batch = int(batch)
        self.dtype = dtype
        self.device = device
        self.group = int(group)
        self.chunk = int(chunk)
        self.num_warps = int(num_warps)
        self.num_stages = int(num_stages)

        n_groups = -(-self.max_len // self.group)
        dshape = (batch, self.num_kv_heads, self.max_len, self.head_dim)
        sshape = (batch, self.num_kv_heads, n_groups, self.head_dim)
        tshape = (batch, self.num_kv_heads, self.group, self.head_dim)
        self.kq = [torch.zeros(dshape, dtype=torch.uint8, device=device) for _ in range(self.num_slots)]
        self.vq = [torch.zeros(dshape, dtype=torch.uint8, device=device) for _ in range(self.num_slots)]
        self.kmn = [torch.zeros(sshape, dtype=dtype, device=device) for _ in range(self.num_slots)]
        self.kst = [torch.zeros(sshape, dtype=dtype, device=device) for _ in range(self.num_slots)]
        self.vmn = [torch.zeros(sshape, dtype=dtype, device=device) for _ in range(self.num_slots)]
        self.vst = [torch.zeros(sshape, dtype=dtype, device=device) for _ in range(self.num_slots)]
        self.tail_k = [torch.zeros(tshape, dtype=dtype, device=device) for _ in range(self.num_slots)]
        self.tail_v = [torch.zeros(tshape, dtype=dtype, device=device) for _ in range(self.num_slots)]

        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        self.first = torch.zeros(1, dtype=torch.long, device=device)
        self._written = torch.zeros(1, dtype=torch.long, device=device)
        self._qlen = torch.zeros(1, dtype=torch.long, device=device)
        self._pg = torch.zeros(1, dtype=torch.long, device=device)
        self._idx64 = torch.arange(self.group, dtype=torch.long, device=device)
        self._arange = torch.arange(self.max_len, dtype=torch.long, device=device)
        self._zero = torch.zeros((), dtype=dtype, device=device)
        self._ninf = torch.full((), float("-inf"), dtype=dtype, device=device)
        self._mask = torch.zeros(self.group, dtype=torch.uint8, device=device)

        # scratch: the reference's shapes. The kernels keep their partials in the workspace
        # `_ws`, whose first bytes `pa` views; `_ws` is zero-filled and serves this cache's
        # decode launches only: the fused step keeps per-head completion counters in its
        # last bytes (every launch leaves them at zero)
        self.n_splits = -(-self.max_len // self.chunk)
        sshape2 = (self.num_kv_heads, self.n_splits, PAD_M)
        self.pm = torch.zeros(sshape2, dtype=torch.float32, device=device)
        self.pl = torch.zeros_like(self.pm)
        pa_numel = self.num_kv_heads * self.n_splits * PAD_M * self.head_dim
        parts = int(_lib.load().nkv_attn_default_parts(self.num_kv_heads, n_groups))
        need = int(_lib.load().nkv_attn_workspace_bytes(self.num_kv_heads, self.num_q_heads, parts))
        self._ws = torch.zeros(max(pa_numel, -(-need // 4)), dtype=torch.float32, device=device)
        self.pa = self._ws[:pa_numel].view(*sshape2, self.head_dim)
        self.out = torch.zeros((batch, self.num_q_heads, 1, self.head_dim), dtype=dtype, device=device)
        self.lse = torch.zeros((batch, self.num_q_heads), dtype=torch.float32, device=device)
        self.merged = torch.zeros((batch, self.num_q_heads, 1, self.head_dim), dtype=dtype, device=device)
        self._n_parts = _pick_parts(self.num_kv_heads, self.num_q_heads, n_groups, self._ws.numel() * 4, fused=True)
        self._ws_bytes = self._ws.numel() * 4

        self.staging: Any = None
        self.stream_chunk = 0
        self._chunk_k: list[torch.Tensor] = []
        self._chunk_v: list[torch.Tensor] = []
        self._chunk_n = [0] * self.num_slots
        self._chunk_off = 0
        self._stream_end: int | None = 0

    # ---- StaticKVCache-compatible surface

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self.pos.item())

    def reset(self) -> None:
        self.pos.zero_()
        self.first.zero_()
        self._written.zero_()
        self._qlen.zero_()
        self._pg.zero_()
        if self.staging is not None:
            self.staging.reset()
        self._stream_end, self._chunk_off = 0, 0

    # ---- prefill: fp16 staging area

    def begin_prefill(self, total_len: int, stream_chunk: int = 0) -> None:
        """Allocate the fp16 staging area for the tokens the prefill will write.

        With ``stream_chunk`` (a multiple of 64) the staging area holds one chunk per layer
        instead of the whole prompt, and every chunk is quantized as it lands."""
        from .cache import StaticKVCache

        total_len = int(total_len)
        if total_len <= 0 or total_len > self.max_len:
            raise ValueError(f"prefill 长度 {total_len} 超出 (0, {self.max_len}]")
        stream_chunk = int(stream_chunk)
        if stream_chunk:
            if stream_chunk < 0 or stream_chunk % self.group:
                raise ValueError(f"块大小 {stream_chunk} 必须是 {self.group} 的整数倍")
            shape = (self.batch, self.num_kv_heads, stream_chunk, self.head_dim)
            if not self._chunk_k or self._chunk_k[0].shape != shape:
                self._chunk_k = [torch.empty(shape, dtype=self.dtype, device=self.device)
                                 for _ in range(self.num_slots)]
                self._chunk_v = [torch.empty_like(t) for t in self._chunk_k]
            self.stream_chunk = stream_chunk
            self._chunk_n = [0] * self.num_slots
            self._chunk_off, self._stream_end = int(self.pos.item()), None
            self.staging = None
            return
        self.stream_chunk = 0
        self.staging = StaticKVCache(
            num_slots=self.num_slots, num_kv_heads=self.num_kv_heads, head_dim=self.head_dim,
            max_len=total_len, batch=self.batch, dtype=self.dtype, device=self.device,
        )

    def set_prefill_pos(self, off: int) -> None:
        self.pos.fill_(int(off))
        if self.stream_chunk:
            off = int(off)
            if self._stream_end is not None and off != self._stream_end:
                raise ValueError(f"流式 prefill 的块必须首尾相接：上一块止于 {self._stream_end}，收到起点 {off}")
            self._chunk_off = off
            self._chunk_n = [0] * self.num_slots
            return
        self._ensure_staging()
        self.staging.pos.fill_(int(off))

    def update(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int):
        """Write K/V. Returns ``(None, None)``: attention goes through ``attend()``.

        With a staging area (prefill) the fp16 staging cache is written; otherwise one
        decode token is appended to the ring and the ring is requantized (HIP launch).
        """
        if self.stream_chunk:
            self._stream_update(key, value, layer_idx)
            return None, None
        if self.staging is not None:
            if key.shape[2] != 1:
                self.staging.append_prefill(key, value, layer_idx)
            else:
                self.staging.update(key, value, layer_idx)
            return None, None
        if key.shape[2] != 1:
            raise RuntimeError("没有暂存区时只支持解码一步（n == 1）；prefill 请先 `begin_prefill()`")
        k, v = self._token(key, "key"), self._token(value, "value")
        _lib.call(
            "nkv_append_t64", k.data_ptr(), v.data_ptr(), k.stride(1), self.kq[layer_idx].data_ptr(),
            self.kmn[layer_idx].data_ptr(), self.kst[layer_idx].data_ptr(), self.vq[layer_idx].data_ptr(),
            self.vmn[layer_idx].data_ptr(), self.vst[layer_idx].data_ptr(), self.tail_k[layer_idx].data_ptr(),
            self.tail_v[layer_idx].data_ptr(), self.pos.data_ptr(), self._written.data_ptr(),
            self._qlen.data_ptr(), self._pg.data_ptr(), self.num_kv_heads, self.head_dim, self.max_len,
            _lib.stream_ptr(self.pos.device))
        return None, None

    append_prefill = update

    def _chunk_view(self, bufs: list[torch.Tensor], layer_idx: int, n: int) -> torch.Tensor:
        """The first ``n`` tokens of a chunk buffer as a contiguous ``[1, H_kv, n, D]``."""
        return bufs[layer_idx].view(-1)[:self.num_kv_heads * n * self.head_dim].view(
            1, self.num_kv_heads, n, self.head_dim)

    def _stream_update(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int) -> None:
        """One chunk of a streamed prefill: keep it in fp16 for its own attention, quantize
        its whole groups into ``[off, off + 64*floor(n/64))`` and put its newest
        ``min(n, 64)`` tokens into the ring (slot = position mod 64)."""
        n, off = key.shape[2], self._chunk_off
        shape = (1, self.num_kv_heads, n, self.head_dim)
        if key.shape != shape or value.shape != shape:
            raise ValueError(f"key / value must be [1, {self.num_kv_heads}, n, {self.head_dim}]")
        if key.dtype != self.dtype or value.dtype != self.dtype:
            raise ValueError(f"key / value 必须是 {self.dtype}")
        if n > self.stream_chunk:
            raise ValueError(f"块长 {n} 超过 stream_chunk {self.stream_chunk}")
        if off % self.group:
            raise ValueError(f"流式 prefill 的块起点 {off} 必须是 {self.group} 的整数倍（只有最后一块可以不满）")
        if off + n > self.max_len:
            raise ValueError(f"prefill 写到 {off + n}，超过 max_len {self.max_len}")
        self._chunk_view(self._chunk_k, layer_idx, n).copy_(key)
        self._chunk_view(self._chunk_v, layer_idx, n).copy_(value)
        self._chunk_n[layer_idx] = n
        q = n // self.group * self.group
        if q:
            g0, g1 = off // self.group, (off + q) // self.group
            for bufs, dq, dmn, dst in ((self._chunk_k, self.kq, self.kmn, self.kst),
                                       (self._chunk_v, self.vq, self.vmn, self.vst)):
                quantize_int8_into(self._chunk_view(bufs, layer_idx, n)[:, :, :q], self.group, dq[layer_idx][:, :, off:off + q],
                                   dmn[layer_idx][:, :, g0:g1], dst[layer_idx][:, :, g0:g1])
        take = min(n, self.group)
        slots = torch.remainder(torch.arange(off + n - take, off + n, device=self.pos.device), self.group)
        self.tail_k[layer_idx].index_copy_(2, slots, key[:, :, n - take:n])
        self.tail_v[layer_idx].index_copy_(2, slots, value[:, :, n - take:n])
        self._stream_end = off + n

    def _token(self, x: torch.Tensor, name: str) -> torch.Tensor:
        if x.shape != (1, self.num_kv_heads, 1, self.head_dim):
            raise ValueError(f"{name} must be [1, {self.num_kv_heads}, 1, {self.head_dim}], got {tuple(x.shape)}")
        if x.dtype != self.dtype:
            raise ValueError(f"{name} 必须是 {self.dtype}，收到 {x.dtype}")
        if x.stride(3) != 1 or x.stride(1) % 8 or x.data_ptr() % 16:
            x = x.contiguous()
        return x

    @property
    def prefilling(self) -> bool:
        """True between ``begin_prefill`` and ``finish_prefill`` (staged or streamed)."""
        return self.staging is not None or bool(self.stream_chunk)

    def _ensure_staging(self) -> None:
        if self.staging is None:
            raise RuntimeError("fp16 暂存区不存在：prefill 前先 `begin_prefill(total_len)`")

    def _sync_scalars(self) -> None:
        """``_written = pos + 1``, ``_qlen`` = whole-group boundary, ``_pg`` = group count
        (device tensor ops; the decode launches set the same values themselves)."""
        self._written.copy_(self.pos)
        self._written.add_(1)
        self._qlen.copy_(self._written)
        self._qlen.div_(self.group, rounding_mode="floor")
        self._qlen.mul_(self.group)
        self._pg.copy_(self._qlen)
        self._pg.div_(self.group, rounding_mode="floor")

    def refresh_scalars(self) -> None:
        """Recompute the device scalars from ``pos`` (outside a graph, after warmup)."""
        self._sync_scalars()

    def finish_prefill(self, total: int) -> None:
        """Quantize whole groups of the staging area (one bulk HIP launch per layer and
        tensor, written straight into the cache), fill the ring with the newest <= 64
        tokens, set the scalars and free the staging area (``kvattn.py:745-783``)."""
        total = int(total)
        q = total // self.group * self.group
        n_groups = q // self.group
        if self.stream_chunk:
            if total != self._stream_end:
                raise ValueError(f"流式 prefill 写到 {self._stream_end}，finish_prefill 收到 {total}")
            self.pos.fill_(total)
            self.first.fill_(0)
            self._written.fill_(total)
            self._qlen.fill_(q)
            self._pg.fill_(n_groups)
            self.stream_chunk = 0
            return
        self._ensure_staging()
        for layer in range(self.num_slots):
            src_k = self.staging.key_cache[layer]
            src_v = self.staging.value_cache[layer]
            if n_groups:
                quantize_int8_into(src_k[:, :, :q], self.group, self.kq[layer][:, :, :q],
                                   self.kmn[layer][:, :, :n_groups], self.kst[layer][:, :, :n_groups])
                quantize_int8_into(src_v[:, :, :q], self.group, self.vq[layer][:, :, :q],
                                   self.vmn[layer][:, :, :n_groups], self.vst[layer][:, :, :n_groups])
            take = min(total, self.group)
            if take:
                slots = torch.remainder(torch.arange(total - take, total, device=self.pos.device), self.group)
                self.tail_k[layer].index_copy_(2, slots, src_k[:, :, total - take:total])
                self.tail_v[layer].index_copy_(2, slots, src_v[:, :, total - take:total])
        self.pos.fill_(total)
        self.first.fill_(0)
        self._written.fill_(total)
        self._qlen.fill_(q)
        self._pg.fill_(n_groups)
        self.staging = None

    def release_staging(self) -> None:
        self.staging = None
        self.stream_chunk = 0
        self._chunk_k, self._chunk_v = [], []

    # ---- prefill attention (fp16 staging + causal mask, as the reference)

    def attend_prefill(self, query: torch.Tensor, layer_idx: int) -> torch.Tensor:
        """Attention of one prefill chunk over ``[0, off+n)`` of the fp16 staging area
        with a causal mask (``kvattn.py:791-815``).

        In a streamed prefill the history ``[0, off)`` is read from the int8 cache and the
        chunk from its fp16 copy (one MFMA launch pair, :func:`int8_prefill_attend`)."""
        if self.stream_chunk:
            n, off = query.shape[2], self._chunk_off
            if n != self._chunk_n[layer_idx]:
                raise RuntimeError(f"layer {layer_idx}: attend_prefill 的块长 {n} 与 update 写入的 "
                                   f"{self._chunk_n[layer_idx]} 不符")
            return int8_prefill_attend(query.contiguous(), self._chunk_view(self._chunk_k, layer_idx, n),
                                       self._chunk_view(self._chunk_v, layer_idx, n), self.kq[layer_idx], self.kmn[layer_idx],
                                       self.kst[layer_idx], self.vq[layer_idx], self.vmn[layer_idx],
                                       self.vst[layer_idx], off)
        self._ensure_staging()
        n = query.shape[2]
        off = int(self.staging.pos.item())
        hist = off + n
        key = self.staging.key_cache[layer_idx][:, :, :hist]
        value = self.staging.value_cache[layer_idx][:, :, :hist]
        gq = self.num_q_heads // self.num_kv_heads
        key = key[:, :, None, :, :].expand(1, self.num_kv_heads, gq, hist, self.head_dim)
        key = key.reshape(1, self.num_q_heads, hist, self.head_dim).contiguous()
        value = value[:, :, None, :, :].expand(1, self.num_kv_heads, gq, hist, self.head_dim)
        value = value.reshape(1, self.num_q_heads, hist, self.head_dim).contiguous()
        rows = off + torch.arange(n, device=query.device)
        keep = self._arange[:hist].view(1, 1, 1, -1) <= rows.view(1, 1, n, 1)
        mask = torch.where(keep, self._zero, self._ninf)
        return F.scaled_dot_product_attention(query.contiguous(), key, value, attn_mask=mask, dropout_p=0.0,
                                              scale=self.head_dim ** -0.5)

    # ---- decode: ring mask / attention

    def ring_mask(self) -> torch.Tensor:
        """Ring validity ``[1,1,1,64]`` bool from the device scalars (HIP launch):
        slot ``i`` holds ``p = u - ((u - i) mod 64)``, ``u = _written - 1``, valid iff
        ``_qlen <= p <= u`` and ``p >= first`` (``kvattn.py:819-833``)."""
        _lib.call("nkv_ring_mask", self._written.data_ptr(), self._qlen.data_ptr(), self.first.data_ptr(),
                  self.group, self._mask.data_ptr(), _lib.stream_ptr(self.pos.device))
        return self._mask.view(1, 1, 1, self.group).bool()

    def _q(self, query: torch.Tensor) -> torch.Tensor:
        if query.shape[2] != 1:
            raise ValueError("attend() 只处理解码一步（q_len == 1）；prefill 走 attend_prefill()")
        if query.shape != (1, self.num_q_heads, 1, self.head_dim) or query.dtype != self.dtype:
            raise ValueError(f"query must be fp16 [1, {self.num_q_heads}, 1, {self.head_dim}], "
                             f"got {tuple(query.shape)} {query.dtype}")
        return query if query.is_contiguous() and query.data_ptr() % 16 == 0 else query.contiguous()

    def attend(self, query: torch.Tensor, layer_idx: int) -> torch.Tensor:
        """Decode-step attention over the int8 prefix and the valid ring slots, one
        softmax (one ``nkv_attn_decode_t64`` call); writes and returns ``merged`` (``lse`` holds the
        log-sum-exp). No host sync — lengths come from ``_qlen`` / ``_pg`` / ``_written``.
        A one-token chunk of a streamed prefill is attended as a chunk."""
        if self.stream_chunk:
            return self.attend_prefill(query, layer_idx)
        q = self._q(query)
        _lib.call(
            "nkv_attn_decode_t64", q.data_ptr(), self.kq[layer_idx].data_ptr(), self.kmn[layer_idx].data_ptr(),
            self.kst[layer_idx].data_ptr(), self.vq[layer_idx].data_ptr(), self.vmn[layer_idx].data_ptr(),
            self.vst[layer_idx].data_ptr(), self.num_q_heads, self.num_kv_heads, self.head_dim, self.max_len,
            0, 0, self._qlen.data_ptr(), self._pg.data_ptr(), self.tail_k[layer_idx].data_ptr(),
            self.tail_v[layer_idx].data_ptr(), self._written.data_ptr(), self.first.data_ptr(),
            self.merged.data_ptr(), self.lse.data_ptr(), self._ws.data_ptr(), self._ws_bytes,
            self._n_parts, _lib.stream_ptr(self.pos.device))
        return self.merged

    def update_attend(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor,
                      layer_idx: int) -> torch.Tensor:
        """``update()`` + ``attend()`` of one decode token in one ``nkv_decode_step_t64`` call.

        Same cache state and scalars as the two calls; the output equals ``attend()``'s up
        to float summation order. During prefill (staging present) it falls back to the
        two-call sequence's staging semantics via ``update`` + ``attend_prefill``.
        """
        if self.prefilling:
            self.update(key, value, layer_idx)
            return self.attend_prefill(query, layer_idx)
        _lib.call("nkv_decode_step_t64", *self.step_args(key, value, query, layer_idx))
        return self.merged

    def step_args(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer_idx: int) -> tuple:
        """Arguments of the decode-step entry points (``nkv_decode_step_t64`` and its two
        halves ``_partials`` / ``_combine``) for one decode token of layer ``layer_idx``
        on the current stream. The tensors must stay alive until the launch completes."""
        if key.shape[2] != 1:
            raise RuntimeError("没有暂存区时只支持解码一步（n == 1）；prefill 请先 `begin_prefill()`")
        k, v = self._token(key, "key"), self._token(value, "value")
        q = self._q(query)
        return (q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(1),
                self.kq[layer_idx].data_ptr(), self.kmn[layer_idx].data_ptr(), self.kst[layer_idx].data_ptr(),
                self.vq[layer_idx].data_ptr(), self.vmn[layer_idx].data_ptr(), self.vst[layer_idx].data_ptr(),
                self.tail_k[layer_idx].data_ptr(), self.tail_v[layer_idx].data_ptr(), self.pos.data_ptr(),
                self.first.data_ptr(), self._written.data_ptr(), self._qlen.data_ptr(), self._pg.data_ptr(),
                self.num_q_heads, self.num_kv_heads, self.head_dim, self.max_len, self.merged.data_ptr(),
                self.lse.data_ptr(), self._ws.data_ptr(), self._ws_bytes, self._n_parts,
                _lib.stream_ptr(self.pos.device))

    # ---- memory accounting

    def set_parts(self, n_parts: int) -> None:
        """Prefix work units per KV head for the decode launches (before any capture); grows
        the workspace when needed (zero-filled)."""
        need = int(_lib.load().nkv_attn_workspace_bytes(self.num_kv_heads, self.num_q_heads, int(n_parts)))
        if need > self._ws.numel() * 4:
            pa_numel = self.pa.numel()
            self._ws = torch.zeros(max(pa_numel, -(-need // 4)), dtype=torch.float32, device=self._ws.device)
            self.pa = self._ws[:pa_numel].view(self.pa.shape)
            self._ws_bytes = self._ws.numel() * 4
        self._n_parts = int(n_parts)

    def nbytes(self) -> int:
        """Resident KV bytes: codes, rulers and ring (no scratch, no staging)."""
        q = sum(t.numel() for t in self.kq) + sum(t.numel() for t in self.vq)
        scales = sum(t.numel() * t.element_size() for t in self.kmn + self.kst + self.vmn + self.vst)
        tail = sum(t.numel() * t.element_size() for t in self.tail_k + self.tail_v)
        return q + scales + tail

    def fp16_nbytes(self) -> int:
        return 2 * self.batch * self.num_slots * self.num_kv_heads * self.max_len * self.head_dim * 2

    def extra_repr(self) -> str:
        return (f"max_len={self.max_len}, slots={self.num_slots}, "
                f"kv={self.nbytes() / 1024 ** 2:.0f}MiB (fp16 {self.fp16_nbytes() / 1024 ** 2:.0f}MiB)")
