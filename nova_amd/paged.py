"""Paged int8 KV cache for a batch of sequences of different lengths (int8t64 format).

The reference serves one sequence at a time (src/nova/kvattn.py:326-327) and pads lengths to
power-of-two buckets with an additive -inf mask (src/nova/decode.py:39-48, 200-205). Here a batch
of ragged sequences shares one page pool per layer:

- a page is one 64-token group of one KV head: K codes (64 x 128 B), V codes, then the four fp16
  rulers ``kst | kmn | vst | vmn`` (128 each) = 17408 bytes, 128-byte aligned;
  ``pages[layer]`` is uint8 ``[num_pages, H_kv, 17408]``;
- ``page_table`` int32 ``[max_seqs, max_pages_per_seq]`` maps a sequence's group ``g`` to a page
  (the same page id in every layer's pool); -1 marks a slot without a page (never reserved, or
  released), and the kernels neither read nor write through it;
- each sequence keeps its own fp16 ring of the newest tokens (``rings[layer]`` fp16
  ``[max_seqs, H_kv, 2, 64, 128]``, K then V) and its write position ``pos[b]``.

A decode step appends one token per sequence (ring write + requantization of the ring into the
sequence's current page) and attends each sequence over exactly its own tokens ``[0, pos_b]``:
the bucket-padded positions the reference masks to -inf are not read, so whatever they hold
cannot change an output. Every computation is a HIP launch (``nkv_paged_decode_step_t64``);
lengths are device scalars, so one captured graph serves every step while pages stay reserved.

``PagedKVInt8TokCache`` holds the per-token symmetric format (one fp16 scale per token and KV
head) in the same page pool scheme: a page is 64 tokens of one KV head, K codes | V codes | K
scales (64 fp16) | V scales = 16640 bytes, 128-byte aligned. It keeps no ring; a decode step is
one launch (``nkv_paged_decode_step_tok``) that stores each sequence's new token into its page and
attends over ``[0, pos_b]``.

Host bookkeeping (``PagePool``: free pages, reservations, lengths; ``plan_parts``: the prefix
work plan) is plain Python so that its guards are testable without a GPU.
"""

from __future__ import annotations

import torch

from . import _lib
from .kvquant import _DT

D = 128
GT = 64
PAGE_BYTES = 2 * GT * D + 4 * D * 2
PAGE_BYTES_TOK = 2 * GT * D + 2 * GT * 2
CODE_BYTES = GT * D
MAX_PARTS_PER_SEQ = 256  # partials the tail's merge holds for one sequence


class PagePool:
    """Which pages each sequence owns, and how far each has written.

    ``reserve`` hands out pages for a sequence's first ``n`` tokens (always from group 0 up, the
    kernels rely on it); ``release`` returns them; ``advance`` records decode steps and refuses one
    that would write past the reserved pages. Table rows to write are returned to the caller."""

    def __init__(self, num_pages: int, max_seqs: int, max_pages_per_seq: int) -> None:
        self.num_pages, self.max_seqs, self.max_pages_per_seq = int(num_pages), int(max_seqs), int(max_pages_per_seq)
        self.free = list(range(self.num_pages - 1, -1, -1))
        self.owned: list[list[int]] = [[] for _ in range(self.max_seqs)]
        self.length = [0] * self.max_seqs

    def _seq(self, b: int) -> int:
        b = int(b)
        if not 0 <= b < self.max_seqs:
            raise ValueError(f"sequence {b} outside [0, {self.max_seqs})")
        return b

    def reserve(self, b: int, n_tokens: int) -> list[tuple[int, int]]:
        """Pages for every group of sequence ``b``'s first ``n_tokens`` tokens; returns the new
        ``(group, page)`` entries of its table row."""
        b = self._seq(b)
        need = -(-int(n_tokens) // GT)
        if need > self.max_pages_per_seq:
            raise ValueError(f"{n_tokens} tokens need {need} pages > max_pages_per_seq {self.max_pages_per_seq}")
        own = self.owned[b]
        if need - len(own) > len(self.free):
            raise RuntimeError(f"page pool exhausted: sequence {b} needs {need - len(own)} more pages, "
                               f"{len(self.free)} are free")
        new = []
        while len(own) < need:
            own.append(self.free.pop())
            new.append((len(own) - 1, own[-1]))
        return new

    def release(self, b: int) -> None:
        b = self._seq(b)
        self.free.extend(reversed(self.owned[b]))
        self.owned[b] = []
        self.length[b] = 0

    def set_length(self, b: int, n: int) -> None:
        b = self._seq(b)
        if n > 0 and (n - 1) // GT >= len(self.owned[b]):
            raise RuntimeError(f"sequence {b}: {n} tokens but only {len(self.owned[b])} pages reserved")
        self.length[b] = int(n)

    def advance(self, seqs: int, steps: int) -> None:
        """``steps`` decode steps of sequences ``0 .. seqs - 1``: each writes tokens at its length;
        the last one written must lie in a reserved page."""
        for b in range(seqs):
            last = self.length[b] + steps - 1
            if last // GT >= len(self.owned[b]):
                raise RuntimeError(f"sequence {b}: {steps} more steps write token {last}, beyond its "
                                   f"{len(self.owned[b])} reserved pages; reserve() more first")
        for b in range(seqs):
            self.length[b] += steps


def plan_parts(lengths: list[int], target_parts: int) -> tuple[list[int], list[int]]:
    """The prefix kernel's work plan: about ``target_parts`` units per KV head split over the
    sequences in proportion to their groups, each sequence at least one and at most
    ``MAX_PARTS_PER_SEQ``. Returns ``(wg_map, seq_parts)``: unit w serves sequence
    ``wg_map[w] >> 16``, part ``wg_map[w] & 0xffff``; ``seq_parts[2b]`` is the first unit of
    sequence b and ``seq_parts[2b + 1]`` its number of parts."""
    if not lengths:
        raise ValueError("no sequences to plan")
    groups = [max(1, int(n) // GT) for n in lengths]
    tot = sum(groups)
    parts = [max(1, min(MAX_PARTS_PER_SEQ, round(target_parts * gr / tot))) for gr in groups]
    wg_map, seq_parts = [], []
    for b, p in enumerate(parts):
        seq_parts += [len(wg_map), p]
        wg_map += [(b << 16) | i for i in range(p)]
    return wg_map, seq_parts


class PagedKVInt8Cache:
    page_bytes = PAGE_BYTES  # bytes of one page of one KV head
    has_rings = True

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, num_q_heads: int, max_seqs: int,
                 num_pages: int, max_pages_per_seq: int, device: str | torch.device = "cuda",
                 target_parts: int | None = None) -> None:
        if head_dim != D:
            raise NotImplementedError(f"head_dim {head_dim}: the HIP kernels are built for {D}")
        if num_q_heads % num_kv_heads or num_q_heads // num_kv_heads > 16:
            raise ValueError(f"Q heads {num_q_heads} / KV heads {num_kv_heads}")
        _lib.load()
        self.num_layers, self.num_kv_heads, self.head_dim = int(num_layers), int(num_kv_heads), int(head_dim)
        self.num_q_heads, self.max_seqs, self.num_pages = int(num_q_heads), int(max_seqs), int(num_pages)
        self.max_pages_per_seq, self.device = int(max_pages_per_seq), device
        self.pool = PagePool(self.num_pages, self.max_seqs, self.max_pages_per_seq)
        self.pages = [torch.zeros((self.num_pages, self.num_kv_heads, self.page_bytes), dtype=torch.uint8,
                                  device=device) for _ in range(self.num_layers)]
        self.rings = ([torch.zeros((self.max_seqs, self.num_kv_heads, 2, GT, D), dtype=torch.float16, device=device)
                       for _ in range(self.num_layers)] if self.has_rings else None)
        self.page_table = torch.full((self.max_seqs, self.max_pages_per_seq), -1, dtype=torch.int32, device=device)
        self.pos = torch.zeros(self.max_seqs, dtype=torch.long, device=device)
        self.merged = torch.zeros((self.max_seqs, self.num_q_heads, 1, D), dtype=torch.float16, device=device)
        self.lse = torch.zeros((self.max_seqs, self.num_q_heads), dtype=torch.float32, device=device)
        self.target_parts = int(target_parts or max(1, 256 // self.num_kv_heads))
        self.wg_map = self.seq_parts = self.ws = None
        self.total_parts = 0
        self.nseq = 0

    # the pool's lists, as attributes (tests hand out pages in a scrambled order through _free)
    @property
    def _free(self) -> list[int]:
        return self.pool.free

    @_free.setter
    def _free(self, ids: list[int]) -> None:
        self.pool.free = list(ids)

    @property
    def _owned(self) -> list[list[int]]:
        return self.pool.owned

    @property
    def _len(self) -> list[int]:
        return self.pool.length

    # ---- pages

    def reserve(self, b: int, n_tokens: int) -> None:
        """Give sequence ``b`` pages for every group of its first ``n_tokens`` tokens."""
        new = self.pool.reserve(b, n_tokens)
        if new:
            g0 = new[0][0]
            ids = torch.tensor([p for _, p in new], dtype=torch.int32)
            self.page_table[b, g0:g0 + len(new)] = ids.to(self.page_table.device)

    def release(self, b: int) -> None:
        """Return sequence ``b``'s pages to the pool; its table row goes back to -1, so a plan that
        still names it appends nothing and attends nothing for it."""
        self.pool.release(b)
        self.page_table[b].fill_(-1)
        self.pos[b] = 0

    # ---- prefill of one sequence

    def _check_prompt(self, key: torch.Tensor, value: torch.Tensor) -> int:
        h = self.num_kv_heads
        for name, x in (("key", key), ("value", value)):
            if x.dim() != 4 or x.shape[0] != 1 or x.shape[1] != h or x.shape[3] != D or x.dtype not in _DT:
                raise ValueError(f"{name} must be [1, {h}, n, {D}] fp16 / bf16 / fp32, got {tuple(x.shape)} {x.dtype}")
        if key.shape != value.shape:
            raise ValueError(f"key {tuple(key.shape)} and value {tuple(value.shape)} differ")
        return key.shape[2]

    def prefill(self, b: int, layer: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Store a prompt of n tokens (``[1, H_kv, n, 128]``) for sequence ``b``: whole groups
        quantized by the HIP quantizer straight into their pages (``nkv_paged_quantize_t64``, the
        int8t64 arithmetic bit for bit), the newest <= 64 tokens into its ring (slot = position
        mod 64)."""
        n = self._check_prompt(key, value)
        h = self.num_kv_heads
        self.reserve(b, n + 1)
        q = n // GT * GT
        if q:
            row = self.page_table[b]
            for which, x in enumerate((key, value)):
                xc = x if x.stride(3) == 1 and x.stride(2) == D and x.data_ptr() % 16 == 0 else x.contiguous()
                _lib.call("nkv_paged_quantize_t64", xc.data_ptr(), _DT[x.dtype], xc.stride(1), h, q, which,
                          self.pages[layer].data_ptr(), row.data_ptr(), 0, self.num_pages, _lib.stream_ptr(row.device))
        take = min(n, GT)
        if take:
            slots = torch.remainder(torch.arange(n - take, n, device=key.device), GT)
            self.rings[layer][b, :, 0].index_copy_(1, slots, key[0, :, n - take:n].to(torch.float16))
            self.rings[layer][b, :, 1].index_copy_(1, slots, value[0, :, n - take:n].to(torch.float16))
        self.pool.set_length(b, n)
        self.pos[b] = n

    # ---- work plan of the prefix kernel

    def plan(self, lengths: list[int] | None = None) -> None:
        """Split the prefix work of the active sequences into work units (about ``target_parts``
        per KV head, proportional to each sequence's groups, at most 256 per sequence) and size
        the workspace. Lengths default to the current ones; a plan stays valid while the lengths
        grow (each unit covers a fixed fraction of its sequence's groups)."""
        lengths = list(self._len if lengths is None else lengths)
        wg_map, seq_parts = plan_parts(lengths, self.target_parts)
        dev = self.page_table.device
        self.wg_map = torch.tensor(wg_map, dtype=torch.int32, device=dev)
        self.seq_parts = torch.tensor(seq_parts, dtype=torch.int32, device=dev)
        self.total_parts = len(wg_map)
        nbytes = int(_lib.load().nkv_paged_workspace_bytes(self.num_kv_heads, self.num_q_heads, self.total_parts))
        if self.ws is None or self.ws.numel() * 4 < nbytes:
            self.ws = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
        self.nseq = len(lengths)

    # ---- decode

    def _step_args(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        n = self.nseq
        if q.shape != (n, self.num_q_heads, 1, D) or k.shape != (n, self.num_kv_heads, 1, D) or k.shape != v.shape:
            raise ValueError("q [B, Hq, 1, 128], k / v [B, Hkv, 1, 128] fp16, B = the planned sequences")
        return q.contiguous(), k.contiguous(), v.contiguous()

    def decode_step(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer: int) -> torch.Tensor:
        """Append one token per sequence at ``pos`` and attend each sequence over ``[0, pos_b]``, in
        one launch (``nkv_paged_decode_step_t64``: the tails append). Returns ``merged[:B]``
        ``[B, Hq, 1, 128]``; ``lse`` holds the log-sum-exp."""
        if self.wg_map is None:
            raise RuntimeError("call plan() before decoding")
        q, k, v = self._step_args(query, key, value)
        _lib.call("nkv_paged_decode_step_t64", q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                  self.pages[layer].data_ptr(), self.page_table.data_ptr(), self.page_table.stride(0), self.num_pages,
                  self.rings[layer].data_ptr(), self.pos.data_ptr(), self.nseq, self.num_q_heads, self.num_kv_heads,
                  D, self.wg_map.data_ptr(), self.seq_parts.data_ptr(), self.total_parts, self.merged.data_ptr(),
                  self.lse.data_ptr(), self.ws.data_ptr(), self.ws.numel() * 4, _lib.stream_ptr(self.pos.device))
        return self.merged[:self.nseq]

    def attend(self, query: torch.Tensor, layer: int) -> torch.Tensor:
        """Attention of each planned sequence over ``[0, pos_b]`` with nothing appended (the
        token at ``pos_b`` read from its ring slot), into ``merged[:B]`` / ``lse``: the second
        launch of ``decode_step`` alone (``nkv_paged_attn_decode_t64``)."""
        if self.wg_map is None:
            raise RuntimeError("call plan() before decoding")
        n = self.nseq
        if query.shape != (n, self.num_q_heads, 1, D):
            raise ValueError("q [B, Hq, 1, 128] fp16, B = the planned sequences")
        q = query.contiguous()
        _lib.call("nkv_paged_attn_decode_t64", q.data_ptr(), self.pages[layer].data_ptr(), self.page_table.data_ptr(),
                  self.page_table.stride(0), self.num_pages, self.rings[layer].data_ptr(), self.pos.data_ptr(), n,
                  self.num_q_heads, self.num_kv_heads, D, self.wg_map.data_ptr(), self.seq_parts.data_ptr(),
                  self.total_parts, self.merged.data_ptr(), self.lse.data_ptr(), self.ws.data_ptr(),
                  self.ws.numel() * 4, _lib.stream_ptr(self.pos.device))
        return self.merged[:n]

    def advance(self) -> None:
        """``pos += 1`` for every planned sequence (device op, graph-safe); refuses a step that
        would take a sequence past its reserved pages."""
        self.note_advanced(1)
        self.pos[:self.nseq].add_(1)

    def note_advanced(self, steps: int) -> None:
        """Host bookkeeping of ``steps`` decode steps that advanced every planned sequence on the
        device (``advance()``, or a replayed graph that adds to ``pos``). Raises when a sequence
        would write past the pages reserved for it."""
        self.pool.advance(self.nseq, steps)


class PagedKVInt8TokCache(PagedKVInt8Cache):
    """A batch of ragged sequences in the per-token symmetric format, in pages of 64 tokens of
    one KV head: K codes int8 ``[64, 128]``, V codes, K scales fp16 ``[64]``, V scales
    (16640 bytes). Codes and scales are those of ``nkv_quantize_tok`` bit for bit, token p of
    sequence b at row ``p % 64`` of page ``page_table[b, p // 64]``. Same pool, table, plan and
    graph-safe ``pos`` as ``PagedKVInt8Cache``; no rings."""

    page_bytes = PAGE_BYTES_TOK
    has_rings = False

    def prefill(self, b: int, layer: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Store a prompt of n tokens (``[1, H_kv, n, 128]``) for sequence ``b``: every token
        quantized by the HIP quantizer straight into its page (``nkv_paged_quantize_tok``)."""
        n = self._check_prompt(key, value)
        h = self.num_kv_heads
        self.reserve(b, n + 1)
        if n:
            row = self.page_table[b]
            for which, x in enumerate((key, value)):
                xc = x if x.stride(3) == 1 and x.stride(2) == D and x.data_ptr() % 16 == 0 else x.contiguous()
                _lib.call("nkv_paged_quantize_tok", xc.data_ptr(), _DT[x.dtype], xc.stride(1), h, n, which,
                          self.pages[layer].data_ptr(), row.data_ptr(), 0, self.num_pages, _lib.stream_ptr(row.device))
        self.pool.set_length(b, n)
        self.pos[b] = n

    def decode_step(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer: int) -> torch.Tensor:
        """Store one token per sequence at ``pos`` and attend each sequence over ``[0, pos_b]``, in
        one launch. Returns ``merged[:B]`` ``[B, Hq, 1, 128]``; ``lse`` holds the log-sum-exp."""
        if self.wg_map is None:
            raise RuntimeError("call plan() before decoding")
        q, k, v = self._step_args(query, key, value)
        _lib.call("nkv_paged_decode_step_tok", q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                  self.pages[layer].data_ptr(), self.page_table.data_ptr(), self.page_table.stride(0), self.num_pages,
                  self.pos.data_ptr(), self.nseq, self.num_q_heads, self.num_kv_heads, D, self.wg_map.data_ptr(),
                  self.seq_parts.data_ptr(), self.total_parts, self.merged.data_ptr(), self.lse.data_ptr(),
                  self.ws.data_ptr(), self.ws.numel() * 4, _lib.stream_ptr(self.pos.device))
        return self.merged[:self.nseq]
