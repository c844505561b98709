"""Paged int8 KV cache for a batch of sequences of different lengths (int8t64 format).

The reference serves one sequence at a time (src/nova/kvattn.py:326-327) and pads
lengths to power-of-two buckets with an additive -inf mask (src/nova/decode.py:39-48,
200-205). Here a batch of ragged sequences shares one page pool per layer:

- a page is one 64-token group of one KV head: K codes (64 x 128 B), V codes, then the
  four fp16 rulers ``kst | kmn | vst | vmn`` (128 each) = 17408 bytes, 128-byte aligned;
  ``pages[layer]`` is uint8 ``[num_pages, H_kv, 17408]``;
- ``page_table`` int32 ``[max_seqs, max_pages_per_seq]`` maps a sequence's group ``g`` to a
  page (the same page id in every layer's pool);
- each sequence keeps its own fp16 ring of the newest tokens (``rings[layer]`` fp16
  ``[max_seqs, H_kv, 2, 64, 128]``, K then V) and its write position ``pos[b]``.

A decode step appends one token per sequence (ring write + requantization of the ring
into the sequence's current page) and attends each sequence over exactly its own tokens
``[0, pos_b]``: the bucket-padded positions the reference masks to -inf are simply not
read. Every computation is a HIP launch (``nkv_paged_decode_step_t64``); lengths are
device scalars, so one captured graph serves every step while pages stay reserved.
"""

from __future__ import annotations

import torch

from . import _lib
from .kvquant import quantize_int8

D = 128
GT = 64
PAGE_BYTES = 2 * GT * D + 4 * D * 2
CODE_BYTES = GT * D


class PagedKVInt8Cache:
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
        self.pages = [torch.zeros((self.num_pages, self.num_kv_heads, PAGE_BYTES), dtype=torch.uint8, device=device)
                      for _ in range(self.num_layers)]
        self.rings = [torch.zeros((self.max_seqs, self.num_kv_heads, 2, GT, D), dtype=torch.float16, device=device)
                      for _ in range(self.num_layers)]
        self.page_table = torch.zeros((self.max_seqs, self.max_pages_per_seq), dtype=torch.int32, device=device)
        self.pos = torch.zeros(self.max_seqs, dtype=torch.long, device=device)
        self.merged = torch.zeros((self.max_seqs, self.num_q_heads, 1, D), dtype=torch.float16, device=device)
        self.lse = torch.zeros((self.max_seqs, self.num_q_heads), dtype=torch.float32, device=device)
        self._free = list(range(self.num_pages - 1, -1, -1))
        self._owned: list[list[int]] = [[] for _ in range(self.max_seqs)]
        self._len = [0] * self.max_seqs
        self.target_parts = int(target_parts or max(1, 256 // self.num_kv_heads))
        self.wg_map = self.seq_parts = self.ws = None
        self.total_parts = 0

    # ---- pages

    def reserve(self, b: int, n_tokens: int) -> None:
        """Give sequence ``b`` pages for every group of its first ``n_tokens`` tokens."""
        need = -(-int(n_tokens) // GT)
        if need > self.max_pages_per_seq:
            raise ValueError(f"{n_tokens} tokens need {need} pages > max_pages_per_seq {self.max_pages_per_seq}")
        own = self._owned[b]
        new = []
        while len(own) < need:
            if not self._free:
                raise RuntimeError("page pool exhausted")
            own.append(self._free.pop())
            new.append(len(own) - 1)
        if new:
            ids = torch.tensor([own[i] for i in new], dtype=torch.int32)
            self.page_table[b, new[0]:new[-1] + 1] = ids.to(self.page_table.device)

    def release(self, b: int) -> None:
        self._free.extend(reversed(self._owned[b]))
        self._owned[b] = []
        self._len[b] = 0
        self.pos[b] = 0

    # ---- prefill of one sequence

    def prefill(self, b: int, layer: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Store a prompt of n tokens (``[1, H_kv, n, 128]`` fp16) for sequence ``b``: whole
        groups quantized into its pages (the HIP quantizer, then a copy into the page
        layout), the newest <= 64 tokens into its ring (slot = position mod 64)."""
        n = key.shape[2]
        self.reserve(b, n + 1)
        q = n // GT * GT
        g = q // GT
        h = self.num_kv_heads
        if g:
            ids = torch.tensor(self._owned[b][:g], dtype=torch.long, device=self.page_table.device)
            page = self.pages[layer]
            for i, x in enumerate((key, value)):
                codes, mins, steps = quantize_int8(x[:, :, :q], GT, "token")
                page[ids, :, i * CODE_BYTES:(i + 1) * CODE_BYTES] = codes[0].reshape(h, g, CODE_BYTES).transpose(0, 1)
                base = 2 * CODE_BYTES + i * 4 * D
                page[ids, :, base:base + 2 * D] = steps[0].contiguous().view(torch.uint8).reshape(h, g, 2 * D).transpose(0, 1)
                page[ids, :, base + 2 * D:base + 4 * D] = mins[0].contiguous().view(torch.uint8).reshape(h, g, 2 * D).transpose(0, 1)
        take = min(n, GT)
        if take:
            slots = torch.remainder(torch.arange(n - take, n, device=key.device), GT)
            self.rings[layer][b, :, 0].index_copy_(1, slots, key[0, :, n - take:n])
            self.rings[layer][b, :, 1].index_copy_(1, slots, value[0, :, n - take:n])
        self._len[b] = n
        self.pos[b] = n

    # ---- work plan of the prefix kernel

    def plan(self, lengths: list[int] | None = None) -> None:
        """Split the prefix work of the active sequences into work units (about
        ``target_parts`` per KV head, proportional to each sequence's groups) and size the
        workspace. Lengths default to the current ones; a plan stays valid while the
        lengths grow (each unit covers a fixed fraction of its sequence's groups)."""
        lengths = list(self._len if lengths is None else lengths)
        groups = [max(1, n // GT) for n in lengths]
        tot = sum(groups)
        parts = [max(1, min(256, round(self.target_parts * gr / tot))) for gr in groups]
        wg_map, seq_parts = [], []
        for b, p in enumerate(parts):
            seq_parts += [len(wg_map), p]
            wg_map += [(b << 16) | i for i in range(p)]
        dev = self.page_table.device
        self.wg_map = torch.tensor(wg_map, dtype=torch.int32, device=dev)
        self.seq_parts = torch.tensor(seq_parts, dtype=torch.int32, device=dev)
        self.total_parts = len(wg_map)
        nbytes = int(_lib.load().nkv_paged_workspace_bytes(self.num_kv_heads, self.num_q_heads, self.total_parts))
        if self.ws is None or self.ws.numel() * 4 < nbytes:
            self.ws = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
        self.nseq = len(lengths)

    # ---- decode

    def _step_args(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer: int):
        n = self.nseq
        if q.shape != (n, self.num_q_heads, 1, D) or k.shape != (n, self.num_kv_heads, 1, D) or k.shape != v.shape:
            raise ValueError("q [B, Hq, 1, 128], k / v [B, Hkv, 1, 128] fp16, B = the planned sequences")
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        return q, k, v

    def decode_step(self, key: torch.Tensor, value: torch.Tensor, query: torch.Tensor, layer: int) -> torch.Tensor:
        """Append one token per sequence at ``pos`` and attend each sequence over ``[0, pos_b]``.
        Returns ``merged[:B]`` ``[B, Hq, 1, 128]``; ``lse`` holds the log-sum-exp."""
        if self.wg_map is None:
            raise RuntimeError("call plan() before decoding")
        q, k, v = self._step_args(query, key, value, layer)
        _lib.call("nkv_paged_decode_step_t64", q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                  self.pages[layer].data_ptr(), self.page_table.data_ptr(), self.page_table.stride(0),
                  self.rings[layer].data_ptr(), self.pos.data_ptr(), self.nseq, self.num_q_heads, self.num_kv_heads,
                  D, self.wg_map.data_ptr(), self.seq_parts.data_ptr(), self.total_parts, self.merged.data_ptr(),
                  self.lse.data_ptr(), self.ws.data_ptr(), self.ws.numel() * 4, _lib.stream_ptr(self.pos.device))
        return self.merged[:self.nseq]

    def advance(self) -> None:
        """``pos += 1`` for every planned sequence (device op, graph-safe)."""
        self.note_advanced(1)
        self.pos[:self.nseq].add_(1)

    def note_advanced(self, steps: int) -> None:
        """Host bookkeeping of ``steps`` decode steps that advanced every planned sequence on the
        device (``advance()``, or a replayed graph that adds to ``pos``). Raises when a sequence
        would write past the pages reserved for it."""
        for b in range(self.nseq):
            if (self._len[b] + steps) // GT >= len(self._owned[b]):
                raise RuntimeError(f"sequence {b}: {steps} more steps reach token {self._len[b] + steps}, beyond "
                                   f"its {len(self._owned[b])} reserved pages; reserve() more first")
        for b in range(self.nseq):
            self._len[b] += steps
