"""Graph-captured greedy decoder over the int8 (or fp16) KV cache.

Mirrors ``GraphDecoder`` (src/nova/decode.py:87-526) for the KV paths this package
builds: one hipGraph replay per generated token, the whole step (embed -> layers ->
lm_head -> argmax written back into ``input_ids`` -> ``pos += 1``) inside the graph,
no host sync inside. With ``quant="int8"`` the cache is :class:`KVInt8Cache` and every
layer's attention is one ``update_attend`` call (two HIP launches). Capacity buckets and the O(max_len) mask row
follow ``decode.py:39-48,200-205``. Sliding-window layers and memory injection are
not part of this path.
"""

from __future__ import annotations

import torch

from .cache import StaticKVCache
from .kvattn import KVInt8Cache

BUCKETS: tuple[int, ...] = (2070, 4096, 8192, 16384, 32768, 65536)


def bucket_for(n: int, buckets: tuple[int, ...] = BUCKETS) -> int:
    """Smallest bucket >= n; beyond the largest bucket, exactly n (``decode.py:42-48``)."""
    n = int(n)
    for b in buckets:
        if n <= b:
            return int(b)
    return n


class GraphDecoder:
    """One decode step captured as a graph.

    Usage::

        dec = GraphDecoder(model, max_len=256, quant="int8")
        dec.prefill(prompt_ids)          # eager
        dec.capture()                    # capture
        for _ in range(n):
            dec.step()                   # one replay = one token
    """

    def __init__(self, model, max_len: int = 256, batch: int = 1, device: str | torch.device = "cuda",
                 dtype: torch.dtype = torch.float16, quant: str = "off") -> None:
        self.model = model
        self.text = model.model
        self.cfg = model.config
        self.max_len = max_len
        self.batch = batch
        self.device = device
        self.dtype = dtype
        if quant not in ("off", "int8"):
            raise ValueError(f"quant 只支持 'off' / 'int8'，收到 {quant!r}")
        self.quant = quant
        if any(self.text.layer_windows):
            raise ValueError("sliding-window layers are not part of this KV path")
        self.swa_window = 0
        cache_cls = KVInt8Cache if quant == "int8" else None
        if cache_cls is not None:
            self.cache = KVInt8Cache(num_slots=self.text.num_cache_layers,
                                     num_kv_heads=self.cfg.num_key_value_heads, head_dim=self.cfg.head_dim,
                                     max_len=max_len, num_q_heads=self.cfg.num_attention_heads, batch=batch,
                                     dtype=dtype, device=device)
        else:
            self.cache = StaticKVCache(num_slots=self.text.num_cache_layers,
                                       num_kv_heads=self.cfg.num_key_value_heads, head_dim=self.cfg.head_dim,
                                       max_len=max_len, batch=batch, dtype=dtype, device=device)
        self.input_ids = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self._arange = torch.arange(max_len, dtype=torch.long, device=device)
        self._zero = torch.zeros((), dtype=dtype, device=device)
        self._ninf = torch.full((), torch.finfo(dtype).min, dtype=dtype, device=device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None
        self._captured = False

    # ---- construction

    @staticmethod
    def _build_mask_table(max_len: int, dtype: torch.dtype, device) -> torch.Tensor:
        """``table[pos]``: 0 for the first ``pos + 1`` columns, ``finfo.min`` elsewhere
        (``decode.py:176-189``). Reference table for the mask-row tests only."""
        neg = torch.finfo(dtype).min
        idx = torch.arange(max_len, device=device)
        keep = idx.view(1, -1) <= idx.view(-1, 1)
        zero = torch.zeros((), dtype=dtype, device=device)
        ninf = torch.full((), neg, dtype=dtype, device=device)
        return torch.where(keep, zero, ninf)

    @classmethod
    def for_length(cls, model, n_tokens: int, reserve: int = 64, **kwargs) -> "GraphDecoder":
        return cls(model, max_len=bucket_for(int(n_tokens) + int(reserve)), **kwargs)

    def _mask_row(self, pos: torch.Tensor) -> torch.Tensor:
        """Additive mask row of ``pos`` (0 up to ``pos``, ``finfo.min`` after), ``[1,1,1,max_len]``."""
        return torch.where(self._arange <= pos, self._zero, self._ninf).view(1, 1, 1, self.max_len)

    # ---- eager prefill

    @torch.inference_mode()
    def prefill(self, input_ids: torch.Tensor, offset: int | None = None, reset: bool = True,
                chunk: int = 0) -> torch.Tensor:
        """Eager prefill of the prompt (``decode.py:224-297``): the int8 cache stages fp16
        K/V, attends causally, then quantizes whole groups in ``finish_prefill``.

        ``chunk`` (int8 cache only, a multiple of 64): feed the prompt in chunks of that many
        tokens as a streamed prefill. Each chunk is quantized as it lands, so the fp16
        staging holds one chunk instead of the prompt, and each chunk attends the int8
        history on MFMA. ``offset`` must then be a multiple of 64."""
        if reset:
            self.cache.reset()
        if offset is None:
            offset = int(self.cache.pos.item())
        offset = int(offset)
        n = input_ids.shape[1]
        if n + offset > self.max_len:
            raise ValueError(f"prompt 长度 {n} + 起点 {offset} 超过 max_len {self.max_len}")
        chunk = int(chunk)
        if chunk and not isinstance(self.cache, KVInt8Cache):
            raise ValueError("chunk= streams the prefill of the int8 cache (quant='int8')")
        if chunk and offset % 64:
            raise ValueError(f"流式 prefill 的起点 {offset} 必须是 64 的整数倍")
        if hasattr(self.cache, "begin_prefill"):
            self.cache.begin_prefill(offset + n, stream_chunk=chunk) if chunk else self.cache.begin_prefill(offset + n)
        step = chunk or n
        out = None
        for c0 in range(0, n, step):
            nc = min(step, n - c0)
            off = offset + c0
            self.cache.pos.fill_(off)
            if hasattr(self.cache, "set_prefill_pos"):
                self.cache.set_prefill_pos(off)
            if off:
                rows = torch.arange(off, off + nc, device=self.cache.pos.device)
                keep = self._arange.view(1, 1, 1, -1) <= rows.view(1, 1, nc, 1)
                mask = torch.where(keep, self._zero, self._ninf)
            else:
                mask = None
            out = self.model(input_ids=input_ids[:, c0:c0 + nc], past_key_values=self.cache, attention_mask=mask,
                             cross_mode="off", logits_to_keep=1)
        if hasattr(self.cache, "finish_prefill"):
            self.cache.finish_prefill(offset + n)
        self.input_ids.copy_(out[:, -1].argmax(-1).view(self.batch, 1))
        self.cache.pos.fill_(offset + n)
        return out

    # ---- the in-graph step

    def _body(self) -> torch.Tensor:
        """One full decode step; no host sync."""
        pos = self.cache.pos
        position_ids = pos.view(1, 1, 1).expand(3, self.batch, 1)
        mask = self._mask_row(pos)
        hidden = self.text(input_ids=self.input_ids, past_key_values=self.cache, position_ids=position_ids,
                           attention_mask=mask, cross_mode="off")
        logits = self.model.lm_head_forward(hidden)
        self.input_ids.copy_(logits[:, -1].argmax(dim=-1, keepdim=True).view(self.batch, 1))
        pos.add_(1)
        return logits

    # ---- int8 live state around the warmup (decode.py:353-377)

    def _save_int8_state(self):
        if self.quant != "int8":
            return None
        c = self.cache
        return (c.pos.clone(), c.first.clone(), c._written.clone(), c._qlen.clone(), c._pg.clone(),
                [t.clone() for t in c.tail_k], [t.clone() for t in c.tail_v])

    def _restore_int8_state(self, saved) -> None:
        if saved is None:
            return
        c = self.cache
        pos, first, written, qlen, pg, tk, tv = saved
        c.pos.copy_(pos)
        c.first.copy_(first)
        c._written.copy_(written)
        c._qlen.copy_(qlen)
        c._pg.copy_(pg)
        for i, t in enumerate(tk):
            c.tail_k[i].copy_(t)
        for i, t in enumerate(tv):
            c.tail_v[i].copy_(t)

    def capture(self, warmup: int = 3, pool=None) -> None:
        """Warm up on a side stream, restore the live state, then capture ``_body``
        (``decode.py:379-442``). Call after ``prefill()``."""
        self.model.eval()
        start = int(self.cache.pos.item())
        saved_ids = self.input_ids.clone()
        if self.quant == "int8":
            self.cache.release_staging()
        saved_i8 = self._save_int8_state()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.inference_mode():
                for _ in range(warmup):
                    self._body()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.cache.pos.fill_(start)
        self.input_ids.copy_(saved_ids)
        self._restore_int8_state(saved_i8)
        if self.quant == "int8":
            self.cache.refresh_scalars()
        g = torch.cuda.CUDAGraph()
        with torch.inference_mode():
            with torch.cuda.graph(g, pool=pool):
                self.logits = self._body()
        self.graph = g
        self._captured = True

    def grow(self, new_max_len: int) -> None:
        """Move the written KV into a larger bucket (fp16 cache only; the int8 cache must be
        built at its final size, ``decode.py:444-501``)."""
        new_max_len = int(new_max_len)
        if new_max_len <= self.max_len:
            return
        if self.quant == "int8":
            raise NotImplementedError(
                "int8 cache 不支持跨桶 grow() (codes, rulers and ring would all move): "
                "build GraphDecoder(model, max_len=..., quant='int8') at the final size")
        used = int(self.cache.pos.item())
        old = self.cache
        new = StaticKVCache(num_slots=old.num_slots, num_kv_heads=self.cfg.num_key_value_heads,
                            head_dim=self.cfg.head_dim, max_len=new_max_len, batch=self.batch,
                            dtype=self.dtype, device=self.device)
        for i in range(new.num_slots):
            new.key_cache[i][:, :, :used] = old.key_cache[i][:, :, :used]
            new.value_cache[i][:, :, :used] = old.value_cache[i][:, :, :used]
        new.pos.fill_(used)
        self.cache = new
        self.max_len = new_max_len
        self._arange = torch.arange(new_max_len, dtype=torch.long, device=self.device)
        self.graph = None
        self._captured = False

    @torch.inference_mode()
    def step(self) -> torch.Tensor:
        if self.graph is None:
            raise RuntimeError("还没 capture() (capture first)")
        self.graph.replay()
        return self.logits

    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, n_new_tokens: int) -> torch.Tensor:
        self.prefill(input_ids)
        if not self._captured:
            self.capture()
        out = [self.input_ids.clone()]
        for _ in range(n_new_tokens - 1):
            self.step()
            out.append(self.input_ids.clone())
        return torch.cat(out, dim=1)

    def extra_repr(self) -> str:
        return f"max_len={self.max_len}, slots={self.text.num_cache_layers}, kv={self.cache.nbytes() / 1024 ** 2:.0f}MiB"
