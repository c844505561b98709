"""int8 KV decode attention and the streaming int8 cache on MI355X — drop-in for ``nova.kvattn``.

Public surface (src/nova/kvattn.py): ``GROUP_T``, ``CHUNK``, ``PAD_M``, ``int8_attn_decode``,
``pack_int8_kv``, ``tail_attend`` and ``KVInt8Cache`` with the attributes and methods its callers
touch. Every computation is a call into ``libnova_kv.so``; nothing here falls back to torch math.

How the work maps onto the library:

- ``int8_attn_decode``: ``nkv_attn_decode_t64``, the split-K prefix kernel then the tail kernel
  (the log-sum-exp combine of the partials).
- ``KVInt8Cache`` during decoding: ``update`` is ``nkv_append_t64`` (ring slot, requantization of
  the ring into the current group, device scalars); ``attend`` is ``nkv_attn_decode_t64`` over the
  int8 prefix *and* the ring in one softmax; ``update_attend`` is both in one launch
  (``nkv_decode_step_t64``), which is what the decode loop calls.
- prefill: ``nkv_quantize_int8`` writes whole groups straight into the cache; ``attend_prefill``
  runs the MFMA chunk kernel (``nkv_prefill_attn_hist_t64``) over the int8 history, the fp16
  history still in staging (staged prefill) and the chunk itself.

Numerics: codes and rulers are bit-exact with ``kvquant.quantize_int8(x, 64, "token")``. Decode
outputs match "dequantize, then softmax attention" within the reference's criterion (2 fp16 ULP
or 1e-5 absolute; the ring joins the same softmax instead of a separate fp16 SDPA and merge).

ValueError messages carry the reference's key terms (解码一步, chunk, group, used, 尺子), which its
tests match.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib
from .kvquant import quantize_int8, quantize_int8_into

GROUP_T = 64  # tokens per ruler of the int8t64 format (src/nova/kvattn.py:103)
CHUNK = 512   # split granularity of the reference; sizes the caller-visible scratch
PAD_M = 16    # query heads per KV head are padded to 16 MFMA rows
HEAD_DIM = 128


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _is_pow2(n: int) -> bool:
    return n > 0 and n & (n - 1) == 0


def _capturing() -> bool:
    return bool(torch.cuda.is_available() and torch.cuda.is_current_stream_capturing())


def _require_gpu_tensor(x: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    """The reference's ``_check`` contract (src/nova/kvattn.py:256-262): on the GPU, of the
    given dtype, contiguous."""
    if not x.is_cuda:
        raise ValueError(f"{name} must live on the GPU (CUDA/HIP device)")
    if x.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ---------------------------------------------------------------- one-call decode attention


@dataclass
class _DecodeGeometry:
    hq: int
    hkv: int
    length: int   # cache capacity L (tokens)
    rulers: int   # ruler groups of the cache, ceil(L / group)


def _decode_geometry(q, kq, kmn, kst, vq, vmn, vst, group: int, chunk: int) -> _DecodeGeometry:
    """Shape and dtype contract of ``int8_attn_decode`` (src/nova/kvattn.py:281-386)."""
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError(f"int8_attn_decode attends one decode step (解码一步): q must be [1, H_q, 1, D], "
                         f"got {tuple(q.shape)}")
    if q.shape[0] != 1:
        raise ValueError(f"batch must be 1 (batch 必须为 1), got {q.shape[0]}")
    want = {"q": (q, torch.float16), "kq": (kq, torch.uint8), "vq": (vq, torch.uint8), "kmn": (kmn, torch.float16),
            "kst": (kst, torch.float16), "vmn": (vmn, torch.float16), "vst": (vst, torch.float16)}
    for name, (t, dt) in want.items():
        _require_gpu_tensor(t, name, dt)
    hq, d = q.shape[1], q.shape[3]
    hkv, length = kq.shape[1], kq.shape[2]
    if vq.shape != kq.shape:
        raise ValueError(f"kq {tuple(kq.shape)} and vq {tuple(vq.shape)} differ in shape")
    if not kmn.shape == kst.shape == vmn.shape == vst.shape:
        raise ValueError("the four rulers (尺子) kmn/kst/vmn/vst must share one shape")
    if kmn.shape[0] != 1 or kmn.shape[1] != hkv or kmn.shape[3] != d or kq.shape[3] != d:
        raise ValueError(f"ruler (尺子) shape {tuple(kmn.shape)} does not fit codes {tuple(kq.shape)}")
    if hq % hkv:
        raise ValueError(f"{hq} query heads do not divide into {hkv} KV heads")
    if hq // hkv > PAD_M:
        raise ValueError(f"{hq // hkv} query heads per KV head exceed the padding limit {PAD_M}")
    if not _is_pow2(d):
        raise ValueError(f"head_dim {d} must be a power of two")
    if not _is_pow2(group):
        raise ValueError(f"group {group} must be a power of two")
    if chunk % group:
        raise ValueError(f"chunk {chunk} must be a whole number of groups of {group}")
    if kmn.shape[2] != _cdiv(length, group):
        raise ValueError(f"{kmn.shape[2]} ruler (尺子) groups for {length} tokens; group {group} needs "
                         f"{_cdiv(length, group)}")
    return _DecodeGeometry(hq, hkv, length, kmn.shape[2])


def _scalar_ok(t) -> bool:
    return t is not None and tuple(t.shape) == (1,) and t.dtype == torch.int64 and t.is_cuda


def _parts_fitting(hkv: int, hq: int, groups: int, capacity_bytes: int | None) -> int:
    """The library's default prefix parts for ``groups`` rulers per head, reduced until their
    partials fit ``capacity_bytes`` (when given)."""
    lib = _lib.load()
    parts = int(lib.nkv_attn_default_parts(hkv, groups))
    if capacity_bytes is None:
        return parts
    while parts > 1 and int(lib.nkv_attn_workspace_bytes(hkv, hq, parts)) > capacity_bytes:
        parts -= 1
    if int(lib.nkv_attn_workspace_bytes(hkv, hq, parts)) > capacity_bytes:
        raise ValueError(f"scratch of {capacity_bytes} bytes holds no partial")
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
    """Fused int8 attention of one decode token (``src/nova/kvattn.py:281-427``).

    ``q`` fp16 ``[1, H_q, 1, D]``; ``kq``/``vq`` uint8 ``[1, H_kv, L, D]``; rulers fp16
    ``[1, H_kv, ceil(L/group), D]``. Tokens ``[0, used)`` are read, at most ``prefix_groups``
    whole rulers of them. ``used_t`` / ``prefix_groups_t`` (device int64 ``[1]``) replace the host
    values and are read inside the kernel, so one captured graph serves every length.
    ``scratch = (pm, pl, pa)`` has the reference's shapes for ``n_splits``; the kernel keeps its
    partials in ``pa``'s memory. Under graph capture ``scratch`` is required (nothing may be
    allocated there). ``num_warps`` / ``num_stages`` are accepted and unused: the HIP kernels'
    launch shapes are fixed. Returns ``out`` fp16 ``[1, H_q, 1, D]``; ``lse_out`` (fp32
    ``[1, H_q]``) receives the log-sum-exp.
    """
    _lib.load()
    geo = _decode_geometry(q, kq, kmn, kst, vq, vmn, vst, group, chunk)
    d = q.shape[3]

    # ---- the length: device scalars (graph-safe) or host integers
    on_device = used_t is not None
    if on_device:
        if not _scalar_ok(used_t):
            raise ValueError(f"used_t must be a CUDA int64 [1] tensor, got {tuple(used_t.shape)} {used_t.dtype}")
        if isinstance(prefix_groups, torch.Tensor) and prefix_groups_t is None:
            prefix_groups_t = prefix_groups
        if not _scalar_ok(prefix_groups_t):
            raise ValueError("prefix_groups_t must be a CUDA int64 [1] tensor alongside used_t")
        used_host, pg_host = 0, 0
    else:
        used_host = geo.length if used is None else int(used)
        if not 0 <= used_host <= geo.length:
            raise ValueError(f"used={used_host} lies outside [0, {geo.length}]")
        if isinstance(prefix_groups, torch.Tensor):
            pg_host = int(prefix_groups.item())  # an eager host value
        else:
            pg_host = int(prefix_groups)
        if pg_host < 0:
            pg_host = _cdiv(used_host, group)
        elif pg_host > geo.rulers:
            raise ValueError(f"prefix_groups={pg_host} exceeds the {geo.rulers} ruler (尺子) groups")

    # ---- outputs
    if out is None:
        out = torch.empty((1, geo.hq, 1, d), dtype=torch.float16, device=q.device)
    elif tuple(out.shape) != (1, geo.hq, 1, d) or out.dtype != torch.float16 or not out.is_cuda:
        raise ValueError(f"out must be fp16 [1, {geo.hq}, 1, {d}] on the GPU, got {tuple(out.shape)} {out.dtype}")
    if lse_out is not None and (tuple(lse_out.shape) != (1, geo.hq) or lse_out.dtype != torch.float32
                                or not lse_out.is_cuda):
        raise ValueError(f"lse_out must be fp32 [1, {geo.hq}] on the GPU, got {tuple(lse_out.shape)} {lse_out.dtype}")

    # ---- partial workspace: the caller's scratch, or a cached per-device buffer
    splits = _cdiv(used_host, chunk) if n_splits is None else int(n_splits)
    if (on_device or used_host) and splits < 1:
        raise ValueError(f"n_splits={splits} must be at least 1")
    groups = geo.rulers if on_device else _cdiv(min(used_host, pg_host * group), group)
    if scratch is not None:
        pm, pl, pa = scratch
        want = (geo.hkv, splits, PAD_M)
        if tuple(pm.shape) != want or tuple(pl.shape) != want or tuple(pa.shape) != (*want, d):
            raise ValueError(f"scratch shapes must be {want} / {(*want, d)} (n_splits={splits}), "
                             f"got {tuple(pm.shape)} / {tuple(pa.shape)}")
        ws, ws_bytes = pa, pa.numel() * pa.element_size()
        parts = _parts_fitting(geo.hkv, geo.hq, groups, ws_bytes)
    else:
        if _capturing():
            raise ValueError("under graph capture int8_attn_decode needs scratch=(pm, pl, pa): "
                             "no workspace may be allocated inside a graph")
        parts = _parts_fitting(geo.hkv, geo.hq, groups, None)
        ws = _lib.workspace(q.device, int(_lib.load().nkv_attn_workspace_bytes(geo.hkv, geo.hq, parts)))
        ws_bytes = ws.numel()
    if group != GROUP_T or d != HEAD_DIM:
        raise NotImplementedError(f"the HIP kernels read {GROUP_T}-token rulers at head_dim {HEAD_DIM} "
                                  f"(group={group}, head_dim={d})")
    _lib.call("nkv_attn_decode_t64", q.data_ptr(), kq.data_ptr(), kmn.data_ptr(), kst.data_ptr(), vq.data_ptr(),
              vmn.data_ptr(), vst.data_ptr(), geo.hq, geo.hkv, d, geo.length, used_host, pg_host,
              _lib.ptr(used_t), _lib.ptr(prefix_groups_t), None, None, None, None, out.data_ptr(),
              _lib.ptr(lse_out), ws.data_ptr(), ws_bytes, parts, _lib.stream_ptr(q.device))
    return out


def pack_int8_kv(k: torch.Tensor, v: torch.Tensor, group: int = GROUP_T):
    """fp16 K/V ``[1, H_kv, n, D]`` -> ``(kq, kmn, kst, vq, vmn, vst)``, each contiguous, by the
    token-axis quantizer (``src/nova/kvattn.py:430-441``)."""
    packed = []
    for x in (k, v):
        packed.extend(t.contiguous() for t in quantize_int8(x, group, "token"))
    return tuple(packed)


def tail_attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tail_mask: torch.Tensor):
    """fp16 attention over the ring and its log-sum-exp (``src/nova/kvattn.py:447-482``).

    ``q`` ``[1, H_q, 1, D]``, ``k``/``v`` ``[1, H_kv, R, D]`` (R <= 64) fp16, ``tail_mask`` bool with
    R entries (True = the slot takes part). Returns ``(out fp16 [1, H_q, 1, D], lse fp32 [1, H_q])``;
    with no slot taking part, out is 0 and lse is -inf.
    """
    hq, hkv = q.shape[1], k.shape[1]
    if hq % hkv:
        raise ValueError(f"{hq} query heads do not divide into {hkv} KV heads")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _require_gpu_tensor(t, name, torch.float16)
    slots, d = k.shape[2], k.shape[3]
    flags = tail_mask.reshape(-1)
    if flags.numel() != slots:
        raise ValueError(f"tail_mask has {flags.numel()} entries for {slots} ring slots")
    flags = flags.to(torch.uint8).contiguous()
    out = torch.empty((1, hq, 1, d), dtype=torch.float16, device=q.device)
    lse = torch.empty((1, hq), dtype=torch.float32, device=q.device)
    _lib.call("nkv_tail_attend", q.data_ptr(), k.data_ptr(), v.data_ptr(), flags.data_ptr(), hq, hkv, d, slots,
              out.data_ptr(), lse.data_ptr(), _lib.stream_ptr(q.device))
    return out, lse


def int8_prefill_attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kq: torch.Tensor,
                        kmn: torch.Tensor, kst: torch.Tensor, vq: torch.Tensor, vmn: torch.Tensor,
                        vst: torch.Tensor, used: int, out: torch.Tensor | None = None,
                        scratch: torch.Tensor | None = None, splits: int = 0) -> torch.Tensor:
    """Causal attention of a prefill chunk over an int8t64 cache and fp16 K/V (MFMA kernels).

    ``query`` ``[1, Hq, n, 128]``. The cache's first ``used`` tokens (a multiple of 64) are int8
    (``kq``/``vq`` ``[1, Hkv, L, 128]``, rulers ``[1, Hkv, ceil(L/64), 128]``). ``key``/``value``
    ``[1, Hkv, m, 128]`` fp16 (``m >= n``, any head stride) follow them: the first ``m - n`` are an
    fp16 history, the last ``n`` the chunk. Query token ``i`` attends the int8 tokens, the fp16
    history and chunk tokens ``0..i`` — what ``KVInt8Cache.attend_prefill`` computes with SDPA over
    its fp16 staging (src/nova/kvattn.py:791-815). Returns ``out`` ``[1, Hq, n, 128]`` fp16.
    """
    _require_gpu_tensor(query, "query", torch.float16)
    for t, nm in ((kq, "kq"), (vq, "vq")):
        _require_gpu_tensor(t, nm, torch.uint8)
    for t, nm in ((kmn, "kmn"), (kst, "kst"), (vmn, "vmn"), (vst, "vst")):
        _require_gpu_tensor(t, nm, torch.float16)
    _, hq, n, d = query.shape
    _, hkv, cap, _ = kq.shape
    m = key.shape[2]
    for t, nm in ((key, "key"), (value, "value")):
        if t.dtype != torch.float16 or not t.is_cuda or t.shape[:2] != (1, hkv) or t.shape[3] != d or t.stride(3) != 1:
            raise ValueError(f"{nm} must be fp16 [1, {hkv}, m, {d}] on the GPU with unit element stride")
        if t.stride(2) != d or t.data_ptr() % 16 or t.stride(1) % 8:
            raise ValueError(f"{nm}: token rows must be contiguous and 16-byte aligned")
    if value.shape != key.shape or value.stride() != key.stride():
        raise ValueError("key and value must have one shape and one layout")
    if m < n:
        raise ValueError(f"{m} fp16 K/V tokens for a chunk of {n} queries")
    if used % GROUP_T or not 0 <= used <= cap:
        raise ValueError(f"used={used} must be a multiple of {GROUP_T} in [0, {cap}]")
    if out is None:
        out = torch.empty_like(query)
    lib = _lib.load()
    if splits <= 0:
        splits = int(lib.nkv_prefill_default_splits(hkv, hq, n, used + (m - n) // GROUP_T * GROUP_T))
    need = int(lib.nkv_prefill_workspace_bytes(hkv, hq, n, splits))
    if scratch is None or scratch.numel() * scratch.element_size() < need:
        if _capturing():
            raise ValueError("under graph capture int8_prefill_attend needs a large enough scratch")
        scratch = _lib.workspace(query.device, need)
    _lib.call("nkv_prefill_attn_hist_t64", query.data_ptr(), n, key.data_ptr(), value.data_ptr(), m,
              key.stride(1), kq.data_ptr(), kmn.data_ptr(), kst.data_ptr(), vq.data_ptr(), vmn.data_ptr(),
              vst.data_ptr(), cap, used, hq, hkv, d, out.data_ptr(), scratch.data_ptr(),
              scratch.numel() * scratch.element_size(), splits, _lib.stream_ptr(query.device))
    return out


# ---------------------------------------------------------------- the streaming cache


@dataclass
class _PrefillPlan:
    """What a running prefill has promised: ``staged`` keeps every token in fp16 until
    ``finish_prefill``; ``streamed`` (``chunk`` > 0) quantizes each chunk as it lands, so chunks
    start on group boundaries and follow one another."""

    total: int
    chunk: int = 0
    start: int = 0                 # first token of the chunk being written
    next_start: int | None = 0     # where the next chunk must start (None: anywhere, first chunk)
    lengths: list = field(default_factory=list)  # per layer: tokens written in the current chunk


class KVInt8Cache:
    r"""Streaming int8 KV cache (``src/nova/kvattn.py:488-880``).

    Per layer it keeps an int8 prefix of whole 64-token groups (uint8 codes ``kq``/``vq``
    ``[1, H_kv, max_len, D]``, fp16 rulers ``kmn``/``kst``/``vmn``/``vst`` ``[1, H_kv,
    ceil(max_len/64), D]``) and a 64-slot fp16 ring ``tail_k``/``tail_v`` of the newest tokens
    (slot = position mod 64). Lengths are device scalars (``pos``, ``first``, ``_written``,
    ``_qlen``, ``_pg``), so one captured decode graph stays valid while the prefix grows.

    Each tensor kind is one allocation for all layers; the per-layer lists are views into it.
    The five scalars are views of one int64 block.

    Decoding, per layer: ``update`` appends the token at ``pos`` (ring slot, requantization of the
    ring into group ``pos // 64``, scalars ``_written = pos + 1``, ``_qlen = 64 floor(_written /
    64)``, ``_pg = _qlen / 64``); ``attend`` attends the prefix ``[0, _qlen)`` and the valid ring
    slots in one softmax; ``update_attend`` does both in one launch.

    Prefill, staged (``begin_prefill(total)``): chunks go to an fp16 staging cache and attend it
    causally; ``finish_prefill`` quantizes the whole groups in bulk, fills the ring and drops the
    staging. Streamed (``begin_prefill(total, stream_chunk=c)``, ``c`` a multiple of 64): each chunk
    starts on a group boundary, its whole groups are quantized as it lands, its newest tokens go
    to the ring, and it attends the int8 history plus itself on MFMA (the 64-multiple chunking of
    ``reports/kv-int8-streaming-cache.md:126-131``). Every group is quantized from the same 64 fp16
    tokens either way, so both leave the same state.
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
        if not _is_pow2(head_dim):
            raise ValueError(f"head_dim {head_dim} must be a power of two")
        if num_q_heads % num_kv_heads:
            raise ValueError(f"{num_q_heads} query heads do not divide into {num_kv_heads} KV heads")
        if num_q_heads // num_kv_heads > PAD_M:
            raise ValueError(f"{num_q_heads // num_kv_heads} query heads per KV head exceed the padding limit {PAD_M}")
        if not _is_pow2(group):
            raise ValueError(f"group {group} must be a power of two")
        if chunk % group:
            raise ValueError(f"chunk {chunk} must be a whole number of groups of {group}")
        if batch != 1:
            raise ValueError(f"batch must be 1 (batch 必须为 1), got {batch}")
        if group != GROUP_T or head_dim != HEAD_DIM or dtype != torch.float16:
            raise NotImplementedError(f"the HIP kernels store fp16 K/V with {GROUP_T}-token rulers at "
                                      f"head_dim {HEAD_DIM}")
        lib = _lib.load()

        self.num_slots, self.num_kv_heads, self.head_dim = int(num_slots), int(num_kv_heads), int(head_dim)
        self.max_len, self.num_q_heads, self.batch = int(max_len), int(num_q_heads), int(batch)
        self.dtype, self.device, self.group, self.chunk = dtype, device, int(group), int(chunk)
        self.num_warps, self.num_stages = int(num_warps), int(num_stages)

        lay, hkv, d = self.num_slots, self.num_kv_heads, self.head_dim
        n_groups = _cdiv(self.max_len, self.group)
        # one allocation per kind, layers as views: codes K|V, rulers kmn|kst|vmn|vst, ring K|V
        self._codes = torch.zeros((2, lay, 1, hkv, self.max_len, d), dtype=torch.uint8, device=device)
        self._rulers = torch.zeros((4, lay, 1, hkv, n_groups, d), dtype=dtype, device=device)
        self._ring = torch.zeros((2, lay, 1, hkv, self.group, d), dtype=dtype, device=device)
        self.kq, self.vq = list(self._codes[0]), list(self._codes[1])
        self.kmn, self.kst, self.vmn, self.vst = (list(self._rulers[i]) for i in range(4))
        self.tail_k, self.tail_v = list(self._ring[0]), list(self._ring[1])

        # device scalars: pos (write cursor), first, written, qlen (int8 prefix), pg (its groups)
        self._scalars = torch.zeros(5, dtype=torch.long, device=device)
        self.pos, self.first, self._written, self._qlen, self._pg = (self._scalars[i:i + 1] for i in range(5))
        self._ring_flags = torch.zeros(self.group, dtype=torch.uint8, device=device)

        # the reference's scratch shapes, and the decode workspace: zero-filled, the partials at
        # its start (``pa`` views them), per-head completion counters of the fused step at its
        # end (every launch leaves them at zero). It serves this cache's decode launches only.
        self.n_splits = _cdiv(self.max_len, self.chunk)
        sshape = (hkv, self.n_splits, PAD_M)
        self.pm = torch.zeros(sshape, dtype=torch.float32, device=device)
        self.pl = torch.zeros_like(self.pm)
        pa_numel = hkv * self.n_splits * PAD_M * d
        parts = int(lib.nkv_attn_default_parts(hkv, n_groups))
        need = int(lib.nkv_attn_workspace_bytes(hkv, self.num_q_heads, parts))
        self._ws = torch.zeros(max(pa_numel, _cdiv(need, 4)), dtype=torch.float32, device=device)
        self._ws_bytes = self._ws.numel() * 4
        self.pa = self._ws[:pa_numel].view(*sshape, d)
        self._n_parts = _parts_fitting(hkv, self.num_q_heads, n_groups, self._ws_bytes)
        self.out = torch.zeros((1, self.num_q_heads, 1, d), dtype=dtype, device=device)
        self.lse = torch.zeros((1, self.num_q_heads), dtype=torch.float32, device=device)
        self.merged = torch.zeros((1, self.num_q_heads, 1, d), dtype=dtype, device=device)

        self.staging = None  # fp16 StaticKVCache of a staged prefill
        self._plan: _PrefillPlan | None = None
        self._chunk_k: torch.Tensor | None = None  # streamed prefill: the current chunk, per layer
        self._chunk_v: torch.Tensor | None = None

    # ---- the StaticKVCache surface the model sees

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self.pos.item())

    def reset(self) -> None:
        self._scalars.zero_()
        if self.staging is not None:
            self.staging.reset()
        if self._plan is not None and self._plan.chunk:
            self._plan.start, self._plan.next_start = 0, 0

    @property
    def stream_chunk(self) -> int:
        """Chunk size of a running streamed prefill (0 otherwise)."""
        return self._plan.chunk if self._plan is not None else 0

    @property
    def prefilling(self) -> bool:
        """True between ``begin_prefill`` and ``finish_prefill``."""
        return self._plan is not None

    # ---- prefill

    def begin_prefill(self, total_len: int, stream_chunk: int = 0) -> None:
        """Start a prefill of ``total_len`` tokens; ``stream_chunk`` (a multiple of 64) streams it."""
        total_len, stream_chunk = int(total_len), int(stream_chunk)
        if not 0 < total_len <= self.max_len:
            raise ValueError(f"prefill length {total_len} outside (0, {self.max_len}]")
        if stream_chunk < 0 or stream_chunk % self.group:
            raise ValueError(f"stream_chunk {stream_chunk} must be a multiple of {self.group}")
        self._plan = _PrefillPlan(total=total_len, chunk=stream_chunk, lengths=[0] * self.num_slots)
        if stream_chunk:
            shape = (self.num_slots, 1, self.num_kv_heads, stream_chunk, self.head_dim)
            if self._chunk_k is None or tuple(self._chunk_k.shape) != shape:
                self._chunk_k = torch.empty(shape, dtype=self.dtype, device=self.device)
                self._chunk_v = torch.empty_like(self._chunk_k)
            self._plan.start, self._plan.next_start = int(self.pos.item()), None
            self.staging = None
            return
        from .cache import StaticKVCache

        self.staging = StaticKVCache(num_slots=self.num_slots, num_kv_heads=self.num_kv_heads,
                                     head_dim=self.head_dim, max_len=total_len, batch=1, dtype=self.dtype,
                                     device=self.device)

    def set_prefill_pos(self, off: int) -> None:
        """Move the write cursor to the start of the next prefill chunk."""
        off = int(off)
        self.pos.fill_(off)
        plan = self._require_plan()
        if plan.chunk:
            if plan.next_start is not None and off != plan.next_start:
                raise ValueError(f"streamed prefill chunks must follow one another: the last one ended at "
                                 f"{plan.next_start}, this one starts at {off}")
            plan.start, plan.lengths = off, [0] * self.num_slots
        else:
            self.staging.pos.fill_(off)

    def _require_plan(self) -> _PrefillPlan:
        if self._plan is None:
            raise RuntimeError("no prefill is running: call begin_prefill(total_len) first "
                               "(fp16 暂存区不存在)")
        return self._plan

    def update(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int):
        """Write K/V; returns ``(None, None)`` (attention goes through ``attend``).

        During a prefill the chunk goes to the staging area (staged) or is quantized into the
        cache (streamed); otherwise one decode token is appended at ``pos`` (HIP launch)."""
        plan = self._plan
        if plan is not None and plan.chunk:
            self._land_chunk(key, value, layer_idx)
        elif plan is not None:
            self.staging.update(key, value, layer_idx)
        else:
            if key.shape[2] != 1:
                raise RuntimeError("outside a prefill only one decode token (n == 1) can be appended; "
                                   "call begin_prefill() first")
            k, v = self._decode_token(key, "key"), self._decode_token(value, "value")
            i = layer_idx
            _lib.call("nkv_append_t64", k.data_ptr(), v.data_ptr(), k.stride(1), self.kq[i].data_ptr(),
                      self.kmn[i].data_ptr(), self.kst[i].data_ptr(), self.vq[i].data_ptr(), self.vmn[i].data_ptr(),
                      self.vst[i].data_ptr(), self.tail_k[i].data_ptr(), self.tail_v[i].data_ptr(),
                      self.pos.data_ptr(), self._written.data_ptr(), self._qlen.data_ptr(), self._pg.data_ptr(),
                      self.num_kv_heads, self.head_dim, self.max_len, _lib.stream_ptr(self.pos.device))
        return None, None

    append_prefill = update

    def _quantize_groups(self, layer: int, k16: torch.Tensor, v16: torch.Tensor, start: int) -> None:
        """Quantize the whole groups of ``k16``/``v16`` (``[1, H_kv, n, D]``, tokens from ``start``,
        a group boundary) straight into the cache."""
        n = k16.shape[2] // self.group * self.group
        if not n:
            return
        g0, g1 = start // self.group, (start + n) // self.group
        for src, codes, mins, steps in ((k16, self.kq, self.kmn, self.kst), (v16, self.vq, self.vmn, self.vst)):
            quantize_int8_into(src[:, :, :n], self.group, codes[layer][:, :, start:start + n],
                               mins[layer][:, :, g0:g1], steps[layer][:, :, g0:g1])

    def _fill_ring(self, layer: int, k16: torch.Tensor, v16: torch.Tensor, end: int) -> None:
        """Copy the newest ``min(n, 64)`` of ``n`` tokens ending at position ``end`` into their ring
        slots (position mod 64)."""
        n = k16.shape[2]
        take = min(n, self.group)
        if not take:
            return
        slots = torch.arange(end - take, end, device=self.pos.device) % self.group
        self.tail_k[layer].index_copy_(2, slots, k16[:, :, n - take:])
        self.tail_v[layer].index_copy_(2, slots, v16[:, :, n - take:])

    def _chunk_tokens(self, layer: int, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        flat = self.num_kv_heads * n * self.head_dim
        shape = (1, self.num_kv_heads, n, self.head_dim)
        return self._chunk_k[layer].reshape(-1)[:flat].view(shape), self._chunk_v[layer].reshape(-1)[:flat].view(shape)

    def _land_chunk(self, key: torch.Tensor, value: torch.Tensor, layer: int) -> None:
        """A streamed chunk: kept in fp16 for its own attention, its whole groups quantized into
        the cache, its newest tokens written to the ring."""
        plan = self._plan
        n, start = key.shape[2], plan.start
        shape = (1, self.num_kv_heads, n, self.head_dim)
        if tuple(key.shape) != shape or tuple(value.shape) != shape:
            raise ValueError(f"key / value must be [1, {self.num_kv_heads}, n, {self.head_dim}]")
        if key.dtype != self.dtype or value.dtype != self.dtype:
            raise ValueError(f"key / value must be {self.dtype}")
        if n > plan.chunk:
            raise ValueError(f"a chunk of {n} tokens exceeds stream_chunk {plan.chunk}")
        if start % self.group:
            raise ValueError(f"streamed chunks start on a group boundary (a multiple of {self.group}); {start} "
                             "is not (only the last chunk may be short)")
        if start + n > self.max_len:
            raise ValueError(f"the prefill would write up to {start + n}, beyond max_len {self.max_len}")
        k16, v16 = self._chunk_tokens(layer, n)
        k16.copy_(key)
        v16.copy_(value)
        plan.lengths[layer] = n
        self._quantize_groups(layer, k16, v16, start)
        self._fill_ring(layer, key, value, start + n)
        plan.next_start = start + n

    def _set_scalars(self, written: int) -> None:
        qlen = written // self.group * self.group
        self._scalars.copy_(torch.tensor([written, 0, written, qlen, qlen // self.group], dtype=torch.long))

    def finish_prefill(self, total: int) -> None:
        """End the prefill at ``total`` tokens: a staged prefill quantizes its whole groups in bulk
        (one HIP launch per layer and tensor, written straight into the cache) and fills the ring
        with the newest <= 64 tokens; both kinds set the scalars (``src/nova/kvattn.py:745-783``)."""
        total = int(total)
        plan = self._require_plan()
        if plan.chunk:
            if total != plan.next_start:
                raise ValueError(f"the streamed prefill wrote up to {plan.next_start}, finish_prefill got {total}")
        else:
            for layer in range(self.num_slots):
                k16 = self.staging.key_cache[layer][:, :, :total]
                v16 = self.staging.value_cache[layer][:, :, :total]
                self._quantize_groups(layer, k16, v16, 0)
                self._fill_ring(layer, k16, v16, total)
            self.staging = None
        self._set_scalars(total)
        self._plan = None

    def release_staging(self) -> None:
        """Drop any prefill state (staging area and streamed-chunk buffers)."""
        self.staging = None
        self._plan = None
        self._chunk_k = self._chunk_v = None

    def attend_prefill(self, query: torch.Tensor, layer_idx: int) -> torch.Tensor:
        """Causal attention of one prefill chunk over everything before it and itself
        (``src/nova/kvattn.py:791-815``), on the MFMA chunk kernel: a streamed chunk reads its
        history from the int8 cache, a staged one from the fp16 staging area."""
        plan = self._require_plan()
        n = query.shape[2]
        i = layer_idx
        if plan.chunk:
            if n != plan.lengths[i]:
                raise RuntimeError(f"layer {i}: attend_prefill got {n} queries, update wrote {plan.lengths[i]}")
            k16, v16 = self._chunk_tokens(i, n)
            used = plan.start
        else:
            end = int(self.staging.pos.item()) + n
            k16 = self.staging.key_cache[i][:, :, :end]
            v16 = self.staging.value_cache[i][:, :, :end]
            used = 0
        return int8_prefill_attend(query.contiguous(), k16, v16, self.kq[i], self.kmn[i], self.kst[i], self.vq[i],
                                   self.vmn[i], self.vst[i], used)

    # ---- decoding

    def refresh_scalars(self) -> None:
        """Recompute ``_written``, ``_qlen``, ``_pg`` from ``pos`` (outside a graph; the decode
        launches set them themselves)."""
        written = self.pos + 1
        self._written.copy_(written)
        self._qlen.copy_(written - written % self.group)
        self._pg.copy_(written // self.group)

    def ring_mask(self) -> torch.Tensor:
        """Valid ring slots as bool ``[1, 1, 1, 64]`` (HIP launch, graph-safe): slot ``i`` holds
        position ``p = u - ((u - i) mod 64)``, ``u = _written - 1``, and is valid iff
        ``_qlen <= p <= u`` and ``p >= first`` (``src/nova/kvattn.py:819-833``)."""
        _lib.call("nkv_ring_mask", self._written.data_ptr(), self._qlen.data_ptr(), self.first.data_ptr(),
                  self.group, self._ring_flags.data_ptr(), _lib.stream_ptr(self.pos.device))
        return self._ring_flags.view(1, 1, 1, self.group).bool()

    def _decode_token(self, x: torch.Tensor, name: str) -> torch.Tensor:
        """One decode token ``[1, H_kv, 1, D]`` as the kernels read it: rows of 128 contiguous
        halves, 16-byte aligned, any head stride that keeps the alignment."""
        if tuple(x.shape) != (1, self.num_kv_heads, 1, self.head_dim) or x.dtype != self.dtype:
            raise ValueError(f"{name} must be {self.dtype} [1, {self.num_kv_heads}, 1, {self.head_dim}], "
                             f"got {tuple(x.shape)} {x.dtype}")
        if x.stride(3) != 1 or x.stride(1) % 8 or x.data_ptr() % 16:
            x = x.contiguous()
        return x

    def _decode_query(self, query: torch.Tensor) -> torch.Tensor:
        if query.shape[2] != 1:
            raise ValueError("attend() handles one decode step (解码一步, q_len == 1); prefill chunks go "
                             "through attend_prefill()")
        if tuple(query.shape) != (1, self.num_q_heads, 1, self.head_dim) or query.dtype != self.dtype:
            raise ValueError(f"query must be {self.dtype} [1, {self.num_q_heads}, 1, {self.head_dim}], "
                             f"got {tuple(query.shape)} {query.dtype}")
        if not query.is_contiguous() or query.data_ptr() % 16:
            query = query.contiguous()
        return query

    def _output(self, out: torch.Tensor | None) -> torch.Tensor:
        if out is None:
            return self.merged
        if (tuple(out.shape) != tuple(self.merged.shape) or out.dtype != self.dtype or not out.is_contiguous()
                or out.data_ptr() % 16 or out.device != self.merged.device):
            raise ValueError(f"out must be a contiguous, 16-byte aligned {self.dtype} tensor of shape "
                             f"{tuple(self.merged.shape)} on {self.merged.device}")
        return out

    def attend(self, query: torch.Tensor, layer_idx: int) -> torch.Tensor:
        """Decode attention over the int8 prefix ``[0, _qlen)`` and the valid ring slots in one
        softmax (``nkv_attn_decode_t64``); writes and returns ``merged``, with the log-sum-exp in
        ``lse``. Lengths come from the device scalars (no host sync). During a prefill a
        one-token chunk is attended as a chunk."""
        if self.prefilling:
            return self.attend_prefill(query, layer_idx)
        q, i = self._decode_query(query), layer_idx
        _lib.call("nkv_attn_decode_t64", q.data_ptr(), self.kq[i].data_ptr(), self.kmn[i].data_ptr(),
                  self.kst[i].data_ptr(), self.vq[i].data_ptr(), self.vmn[i].data_ptr(), self.vst[i].data_ptr(),
                  self.num_q_heads, self.num_kv_heads, self.head_dim, self.max_len, 0, 0, self._qlen.data_ptr(),
                  self._pg.data_ptr(), self.tail_k[i].data_ptr(), self.tail_v[i].data_ptr(),
                  self._written.data_ptr(), self.first.data_ptr(), self.merged.data_ptr(), self.lse.data_ptr(),
                  self._ws.data_ptr(), self._ws_bytes, self._n_parts, _lib.stream_ptr(self.pos.device))
        return self.merged

    def step_args(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer_idx: int,
                  out: torch.Tensor | None = None) -> tuple:
        """The argument tuple of the decode-step entry points (``nkv_decode_step_t64`` and its two
        halves) for one token of layer ``layer_idx`` on the current stream. The tensors passed in
        must stay alive until the launch completes."""
        if key.shape[2] != 1:
            raise RuntimeError("outside a prefill only one decode token (n == 1) can be appended; "
                               "call begin_prefill() first")
        k, v = self._decode_token(key, "key"), self._decode_token(value, "value")
        q, o, i = self._decode_query(query), self._output(out), layer_idx
        return (q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(1), self.kq[i].data_ptr(),
                self.kmn[i].data_ptr(), self.kst[i].data_ptr(), self.vq[i].data_ptr(), self.vmn[i].data_ptr(),
                self.vst[i].data_ptr(), self.tail_k[i].data_ptr(), self.tail_v[i].data_ptr(), self.pos.data_ptr(),
                self.first.data_ptr(), self._written.data_ptr(), self._qlen.data_ptr(), self._pg.data_ptr(),
                self.num_q_heads, self.num_kv_heads, self.head_dim, self.max_len, o.data_ptr(),
                self.lse.data_ptr(), self._ws.data_ptr(), self._ws_bytes, self._n_parts,
                _lib.stream_ptr(self.pos.device))

    def update_attend(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer_idx: int,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """``update`` + ``attend`` of one decode token in one launch (``nkv_decode_step_t64``): the
        same cache state and scalars as the two calls, the same output up to float summation
        order. The output goes to ``out`` when given (an fp16 ``[1, H_q, 1, D]`` buffer), else to
        ``merged``. During a prefill it is ``update`` followed by ``attend_prefill``."""
        if self.prefilling:
            self.update(key, value, layer_idx)
            return self.attend_prefill(query, layer_idx)
        args = self.step_args(key, value, query, layer_idx, out)
        _lib.call("nkv_decode_step_t64", *args)
        return self._output(out)

    def update_attend_block(self, x: torch.Tensor, w_qkv: torch.Tensor, x_gamma: torch.Tensor, x_eps: float,
                            q_gamma: torch.Tensor, k_gamma: torch.Tensor, qk_eps: float, inv_freq: torch.Tensor,
                            w_o: torch.Tensor, layer_idx: int, out: torch.Tensor | None = None,
                            h1_out: torch.Tensor | None = None, qkv_out: torch.Tensor | None = None) -> torch.Tensor:
        """``update_attend_qkv`` plus the block's output projection and residual add in the same
        launch: returns ``h1 = x + w_o @ o`` (fp16 ``[hidden]``, into ``h1_out`` when given, which
        may be ``x`` itself), ``o`` being the attention output (also written to ``out``). ``w_o``:
        ``[hidden, H_q D]`` fp16. The same bits as ``update_attend_qkv`` followed by
        ``gemv.rms_gemv(o, w_o, residual=x)``."""
        hidden = x.numel()
        if w_o.dtype != torch.float16 or not w_o.is_contiguous() or w_o.device != self.pos.device \
                or tuple(w_o.shape) != (hidden, self.num_q_heads * self.head_dim):
            raise ValueError(f"w_o must be a contiguous fp16 [{hidden}, {self.num_q_heads * self.head_dim}] tensor "
                             f"on {self.pos.device}")
        if h1_out is None:
            h1_out = torch.empty_like(x)
        if h1_out.dtype != torch.float16 or not h1_out.is_contiguous() or h1_out.numel() != hidden:
            raise ValueError(f"h1_out must be a contiguous fp16 tensor of {hidden} elements")
        self._qkv_step(x, w_qkv, x_gamma, x_eps, q_gamma, k_gamma, qk_eps, inv_freq, layer_idx, out, qkv_out, w_o,
                       h1_out)
        return h1_out

    def update_attend_qkv(self, x: torch.Tensor, w_qkv: torch.Tensor, x_gamma: torch.Tensor, x_eps: float,
                          q_gamma: torch.Tensor, k_gamma: torch.Tensor, qk_eps: float, inv_freq: torch.Tensor,
                          layer_idx: int, out: torch.Tensor | None = None,
                          qkv_out: torch.Tensor | None = None) -> torch.Tensor:
        """One decode token of a decoder layer's attention block in one launch
        (``nkv_decode_step_qkv_t64``): ``qkv = w_qkv @ rms_norm(x, x_gamma)`` (the stacked q, k, v
        projection of ``LeanAttention``, src/nova/layers.py:99-137), the per-head q / k RMSNorm and
        the rotary embedding at ``self.pos`` (``inv_freq``: fp32 ``[D / 2]``), then ``update`` +
        ``attend`` of the token. The same bits as ``nkv_gemv`` + ``nkv_qk_norm_rope`` +
        ``update_attend``. ``x``: fp16 ``[hidden]`` (hidden a multiple of 8, at most 3072);
        ``w_qkv``: ``[(H_q + 2 H_kv) D, hidden]``; ``qkv_out`` (optional, fp16 ``[(H_q + 2 H_kv) D]``)
        receives the normalized, rotated q and k and v."""
        return self._qkv_step(x, w_qkv, x_gamma, x_eps, q_gamma, k_gamma, qk_eps, inv_freq, layer_idx, out, qkv_out,
                              None, None)

    def _qkv_step(self, x, w_qkv, x_gamma, x_eps, q_gamma, k_gamma, qk_eps, inv_freq, layer_idx, out, qkv_out, w_o,
                  h1_out) -> torch.Tensor:
        if self.prefilling:
            raise RuntimeError("update_attend_qkv decodes one token; finish the prefill first")
        hq, hkv, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        rows = (hq + 2 * hkv) * d
        for name, t in (("x", x), ("x_gamma", x_gamma), ("w_qkv", w_qkv), ("q_gamma", q_gamma), ("k_gamma", k_gamma)):
            if t.dtype != torch.float16 or not t.is_contiguous() or t.device != self.pos.device:
                raise ValueError(f"{name} must be a contiguous fp16 tensor on {self.pos.device}")
        hidden = x.numel()
        if tuple(w_qkv.shape) != (rows, hidden) or x_gamma.numel() != hidden:
            raise ValueError(f"w_qkv must be [{rows}, {hidden}] and x_gamma [{hidden}] for x of {hidden} elements")
        if q_gamma.numel() != d or k_gamma.numel() != d:
            raise ValueError(f"q_gamma and k_gamma must have {d} elements")
        if inv_freq.dtype != torch.float32 or not inv_freq.is_contiguous() or inv_freq.numel() != d // 2:
            raise ValueError(f"inv_freq must be a contiguous fp32 tensor of {d // 2} elements")
        if qkv_out is not None and (qkv_out.dtype != torch.float16 or not qkv_out.is_contiguous()
                                    or qkv_out.numel() != rows):
            raise ValueError(f"qkv_out must be a contiguous fp16 tensor of {rows} elements")
        lib = _lib.load()
        need = int(lib.nkv_decode_step_qkv_workspace_bytes(hkv, hq, self.max_len, self._n_parts))
        if need > self._ws_bytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("update_attend_qkv: call it once outside graph capture (its workspace grows)")
            ws = torch.zeros(max(self.pa.numel(), _cdiv(need, 4)), dtype=torch.float32, device=self._ws.device)
            self._ws, self._ws_bytes = ws, ws.numel() * 4
            self.pa = ws[:self.pa.numel()].view(self.pa.shape)
        o, i = self._output(out), layer_idx
        _lib.call("nkv_decode_step_qkv_t64", x.data_ptr(), x_gamma.data_ptr(), float(x_eps), w_qkv.data_ptr(), hidden,
                  q_gamma.data_ptr(), k_gamma.data_ptr(), float(qk_eps), inv_freq.data_ptr(), _lib.ptr(qkv_out),
                  self.kq[i].data_ptr(), self.kmn[i].data_ptr(), self.kst[i].data_ptr(), self.vq[i].data_ptr(),
                  self.vmn[i].data_ptr(), self.vst[i].data_ptr(), self.tail_k[i].data_ptr(), self.tail_v[i].data_ptr(),
                  self.pos.data_ptr(), self.first.data_ptr(), self._written.data_ptr(), self._qlen.data_ptr(),
                  self._pg.data_ptr(), hq, hkv, d, self.max_len, o.data_ptr(), self.lse.data_ptr(), _lib.ptr(w_o),
                  _lib.ptr(h1_out), self._ws.data_ptr(), self._ws_bytes, self._n_parts, _lib.stream_ptr(self.pos.device))
        return o

    def set_parts(self, n_parts: int) -> None:
        """Prefix work units per KV head of the decode launches (before any capture); grows the
        zero-filled workspace when needed, and zero-fills it (the fused projection step's tagged
        words move with the partials' size)."""
        n_parts = int(n_parts)
        need = int(_lib.load().nkv_attn_workspace_bytes(self.num_kv_heads, self.num_q_heads, n_parts))
        if need > self._ws_bytes:
            ws = torch.zeros(max(self.pa.numel(), _cdiv(need, 4)), dtype=torch.float32, device=self._ws.device)
            self._ws, self._ws_bytes = ws, ws.numel() * 4
            self.pa = ws[:self.pa.numel()].view(self.pa.shape)
        else:
            self._ws.zero_()
        self._n_parts = n_parts

    # ---- memory accounting

    def nbytes(self) -> int:
        """Resident KV bytes: codes, rulers and ring (no scratch, no staging)."""
        return sum(t.numel() * t.element_size() for t in (self._codes, self._rulers, self._ring))

    def fp16_nbytes(self) -> int:
        """Bytes of an fp16 cache of the same shape."""
        return 2 * self.num_slots * self.num_kv_heads * self.max_len * self.head_dim * 2

    def extra_repr(self) -> str:
        return (f"max_len={self.max_len}, slots={self.num_slots}, kv={self.nbytes() / 2 ** 20:.0f}MiB "
                f"(fp16 {self.fp16_nbytes() / 2 ** 20:.0f}MiB)")
