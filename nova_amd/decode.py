"""Graph-captured greedy decoding over the int8 (or fp16) KV cache — drop-in for ``nova.decode``.

One replay of a captured graph generates one token: embedding, every layer (with the int8
cache, one ``update_attend`` launch per layer), lm_head, argmax written back into
``input_ids`` and ``pos += 1``, with no host synchronization inside. The surface follows
``GraphDecoder`` (src/nova/decode.py:87-526): ``prefill`` / ``capture`` / ``step`` /
``generate`` / ``grow``, the capacity buckets ``bucket_for`` (``decode.py:39-48``) and the
O(max_len) additive mask row (``decode.py:200-205``), and ``capture(pool=...)`` with the
reference's graph-pool choices (``decode.py:55-86, 379-442``). Sliding-window layers and memory
injection are not part of this path.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass

import torch

from .cache import StaticKVCache
from .kvattn import KVInt8Cache

BUCKETS: tuple[int, ...] = (2070, 4096, 8192, 16384, 32768, 65536)


def bucket_for(n: int, buckets: tuple[int, ...] = BUCKETS) -> int:
    """The smallest bucket holding ``n`` tokens; past the largest bucket, ``n`` itself
    (``src/nova/decode.py:42-48``)."""
    n = int(n)
    return next((int(b) for b in buckets if n <= b), n)


# ---------------------------------------------------------------- graph memory pools


class _PoolRegistry:
    """One graph memory pool shared by captures that ask for it (``src/nova/decode.py:55-86``).

    ``pool="shared"`` always returns the same pool. ``pool="auto"`` returns it while a graph that
    was captured into it is still alive and starts a fresh one otherwise (reusing the pool of a
    destroyed graph is what torch's caching allocator rejects)."""

    def __init__(self) -> None:
        self.handle = None
        self.users: list[weakref.ref] = []

    def live_users(self) -> int:
        self.users = [w for w in self.users if w() is not None]
        return len(self.users)

    def pool(self, fresh_if_idle: bool):
        if self.handle is None or (fresh_if_idle and self.live_users() == 0):
            self.handle = torch.cuda.graph_pool_handle()
        return self.handle

    def register(self, graph) -> None:
        self.users.append(weakref.ref(graph))


_POOLS = _PoolRegistry()


def shared_graph_pool(fresh_if_idle: bool = True):
    """The shared graph pool (``fresh_if_idle``: a new one when no graph uses the current one)."""
    return _POOLS.pool(fresh_if_idle)


def register_pool_user(graph) -> None:
    """Record that ``graph`` was captured into the shared pool (weakly referenced)."""
    _POOLS.register(graph)


def resolve_pool(pool):
    """``capture(pool=...)``'s argument -> what ``torch.cuda.graph`` takes: ``"off"`` (or
    ``None``) -> no pool, ``"auto"`` / ``"shared"`` -> the shared pool, anything else -> itself (a
    handle). The second value says whether the graph must be registered as a user of the pool."""
    if pool is None or (isinstance(pool, str) and pool == "off"):
        return None, False
    if isinstance(pool, str):
        if pool not in ("auto", "shared"):
            raise ValueError(f"pool must be 'off', 'auto', 'shared' or a pool handle, got {pool!r}")
        return shared_graph_pool(fresh_if_idle=pool == "auto"), True
    return pool, False


# ---------------------------------------------------------------- live int8 state around the warmup


@dataclass
class _Int8Snapshot:
    """What a warmup replay changes in an int8 cache and a later replay reads: the device
    scalars and the rings (the codes a warmup writes are rewritten by the next real appends,
    which requantize the whole ring into the group)."""

    scalars: torch.Tensor
    ring: torch.Tensor

    @classmethod
    def take(cls, cache: KVInt8Cache) -> "_Int8Snapshot":
        return cls(cache._scalars.clone(), cache._ring.clone())

    def put_back(self, cache: KVInt8Cache) -> None:
        cache._scalars.copy_(self.scalars)
        cache._ring.copy_(self.ring)


_CACHES = {"off": StaticKVCache, "int8": KVInt8Cache}


class GraphDecoder:
    """One decode step captured as a graph::

        dec = GraphDecoder(model, max_len=256, quant="int8")
        dec.prefill(prompt_ids)     # eager
        dec.capture()               # capture once
        for _ in range(n):
            dec.step()              # one replay = one token
    """

    def __init__(self, model, max_len: int = 256, batch: int = 1, device: str | torch.device = "cuda",
                 dtype: torch.dtype = torch.float16, quant: str = "off") -> None:
        if quant not in _CACHES:
            raise ValueError(f"quant must be one of {sorted(_CACHES)} (quant 只支持 'off' / 'int8'), got {quant!r}")
        text = model.model
        if any(text.layer_windows):
            raise ValueError("sliding-window layers are not part of this KV path")
        self.model, self.text, self.cfg = model, text, model.config
        self.max_len, self.batch, self.device, self.dtype, self.quant = int(max_len), batch, device, dtype, quant
        self.swa_window = 0
        geometry = dict(num_slots=text.num_cache_layers, num_kv_heads=self.cfg.num_key_value_heads,
                        head_dim=self.cfg.head_dim, max_len=self.max_len, batch=batch, dtype=dtype, device=device)
        if quant == "int8":
            geometry["num_q_heads"] = self.cfg.num_attention_heads
        self.cache = _CACHES[quant](**geometry)
        self.input_ids = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self._set_mask_constants(self.max_len)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None
        self._captured = False

    def _set_mask_constants(self, max_len: int) -> None:
        self._arange = torch.arange(max_len, dtype=torch.long, device=self.device)
        self._zero = torch.zeros((), dtype=self.dtype, device=self.device)
        self._ninf = torch.full((), torch.finfo(self.dtype).min, dtype=self.dtype, device=self.device)

    # ---- masks and buckets

    @staticmethod
    def _build_mask_table(max_len: int, dtype: torch.dtype, device) -> torch.Tensor:
        """``[max_len, max_len]``: row ``p`` is 0 on columns ``<= p`` and ``finfo(dtype).min``
        after (``src/nova/decode.py:176-189``); kept only as the reference the mask row is
        checked against."""
        col = torch.arange(max_len, device=device)
        return torch.full((max_len, max_len), torch.finfo(dtype).min, dtype=dtype, device=device).masked_fill(
            col[None, :] <= col[:, None], 0)

    @classmethod
    def for_length(cls, model, n_tokens: int, reserve: int = 64, **kwargs) -> "GraphDecoder":
        """A decoder whose capacity is the bucket of ``n_tokens + reserve``."""
        return cls(model, max_len=bucket_for(int(n_tokens) + int(reserve)), **kwargs)

    def _mask_row(self, pos: torch.Tensor) -> torch.Tensor:
        """The additive mask of the token at ``pos`` as ``[1, 1, 1, max_len]``: 0 up to ``pos``,
        ``finfo.min`` after (``src/nova/decode.py:200-205``), built from device tensors only."""
        keep = self._arange <= pos
        return torch.where(keep, self._zero, self._ninf).view(1, 1, 1, self.max_len)

    # ---- prefill (eager)

    def _prefill_chunks(self, n: int, offset: int, chunk: int):
        """``(start within the prompt, length, absolute position)`` of each forward pass."""
        size = chunk or n
        for c0 in range(0, n, size):
            yield c0, min(size, n - c0), offset + c0

    def _chunk_mask(self, at: int, n: int) -> torch.Tensor | None:
        """The additive causal mask of ``n`` tokens at positions ``at ..`` over the whole cache."""
        if not at:
            return None
        rows = torch.arange(at, at + n, device=self._arange.device)
        return torch.where(self._arange[None, None, None, :] <= rows[None, None, :, None], self._zero, self._ninf)

    @torch.inference_mode()
    def prefill(self, input_ids: torch.Tensor, offset: int | None = None, reset: bool = True,
                chunk: int = 0) -> torch.Tensor:
        """Run the prompt eagerly (``src/nova/decode.py:224-297``) and leave the next token in
        ``input_ids``. With the int8 cache the prompt is staged in fp16 and quantized at the end;
        ``chunk`` (a multiple of 64, int8 only) streams it instead: each chunk is quantized as it
        lands and attends the int8 history on MFMA, and ``offset`` must then be a multiple of 64.
        Returns the logits of the last forward pass."""
        cache = self.cache
        if reset:
            cache.reset()
        offset = int(cache.pos.item()) if offset is None else int(offset)
        n, chunk = input_ids.shape[1], int(chunk)
        if offset + n > self.max_len:
            raise ValueError(f"prompt of {n} tokens from position {offset} exceeds max_len {self.max_len}")
        int8 = isinstance(cache, KVInt8Cache)
        if chunk and not int8:
            raise ValueError("chunk= streams the prefill of the int8 cache (quant='int8')")
        if chunk and offset % 64:
            raise ValueError(f"a streamed prefill starts on a group boundary; offset {offset} is not a multiple of 64")
        if int8:
            cache.begin_prefill(offset + n, stream_chunk=chunk)
        logits = None
        for c0, m, at in self._prefill_chunks(n, offset, chunk):
            cache.pos.fill_(at)
            if int8:
                cache.set_prefill_pos(at)
            logits = self.model(input_ids=input_ids[:, c0:c0 + m], past_key_values=cache,
                                attention_mask=self._chunk_mask(at, m), cross_mode="off", logits_to_keep=1)
        if int8:
            cache.finish_prefill(offset + n)
        self.input_ids.copy_(logits[:, -1].argmax(-1).view(self.batch, 1))
        cache.pos.fill_(offset + n)
        return logits

    # ---- the captured step

    def _body(self) -> torch.Tensor:
        """One decode step on device tensors only (what a replay runs)."""
        pos = self.cache.pos
        hidden = self.text(input_ids=self.input_ids, past_key_values=self.cache,
                           position_ids=pos.view(1, 1, 1).expand(3, self.batch, 1),
                           attention_mask=self._mask_row(pos), cross_mode="off")
        logits = self.model.lm_head_forward(hidden)
        self.input_ids.copy_(logits[:, -1].argmax(dim=-1).view(self.batch, 1))
        pos.add_(1)
        return logits

    def _save_int8_state(self) -> _Int8Snapshot | None:
        """Snapshot of the int8 cache's live state (``src/nova/decode.py:353-377``); None for fp16."""
        return _Int8Snapshot.take(self.cache) if self.quant == "int8" else None

    def _restore_int8_state(self, saved: _Int8Snapshot | None) -> None:
        if saved is not None:
            saved.put_back(self.cache)

    def capture(self, warmup: int = 3, pool: str | object = "off") -> None:
        """Capture ``_body`` after ``warmup`` eager steps on a side stream, with the cache and
        ``input_ids`` put back as they were (``src/nova/decode.py:379-442``). Call after
        ``prefill()``. ``pool``: ``"off"`` (each graph its own memory), ``"auto"`` (share one pool
        while a graph using it lives), ``"shared"`` (always that pool) or a pool handle."""
        handle, shared = resolve_pool(pool)
        self.model.eval()
        start = int(self.cache.pos.item())
        ids = self.input_ids.clone()
        if self.quant == "int8":
            self.cache.release_staging()
        snapshot = self._save_int8_state()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(warmup):
                self._body()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.cache.pos.fill_(start)
        self.input_ids.copy_(ids)
        self._restore_int8_state(snapshot)
        if self.quant == "int8":
            self.cache.refresh_scalars()
        graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(graph, pool=handle):
            self.logits = self._body()
        if shared:
            register_pool_user(graph)
        self.graph, self._captured = graph, True

    def grow(self, new_max_len: int) -> None:
        """Move the written tokens into a larger bucket (``src/nova/decode.py:444-501``): fp16
        cache only. The int8 cache's codes, rulers and ring would all move, so it must be built at
        its final size (NotImplementedError, as in the reference)."""
        new_max_len = int(new_max_len)
        if new_max_len <= self.max_len:
            return
        if self.quant == "int8":
            raise NotImplementedError("the int8 cache does not grow across buckets (int8 cache 不支持跨桶 grow()): "
                                      "build GraphDecoder(model, max_len=..., quant='int8') at its final size")
        used = int(self.cache.pos.item())
        old = self.cache
        new = StaticKVCache(num_slots=old.num_slots, num_kv_heads=self.cfg.num_key_value_heads,
                            head_dim=self.cfg.head_dim, max_len=new_max_len, batch=self.batch, dtype=self.dtype,
                            device=self.device)
        for dst, src in zip(new.key_cache + new.value_cache, old.key_cache + old.value_cache):
            dst[:, :, :used].copy_(src[:, :, :used])
        new.pos.fill_(used)
        self.cache, self.max_len = new, new_max_len
        self._set_mask_constants(new_max_len)
        self.graph, self._captured = None, False

    @torch.inference_mode()
    def step(self) -> torch.Tensor:
        """Generate one token (one replay); returns the captured logits buffer."""
        if self.graph is None:
            raise RuntimeError("capture() must run before step() (还没 capture())")
        self.graph.replay()
        return self.logits

    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, n_new_tokens: int) -> torch.Tensor:
        """Prefill ``input_ids`` and generate ``n_new_tokens`` greedy tokens ``[batch, n]``."""
        self.prefill(input_ids)
        if not self._captured:
            self.capture()
        tokens = [self.input_ids.clone()]
        for _ in range(n_new_tokens - 1):
            self.step()
            tokens.append(self.input_ids.clone())
        return torch.cat(tokens, dim=1)

    def extra_repr(self) -> str:
        return f"max_len={self.max_len}, slots={self.text.num_cache_layers}, kv={self.cache.nbytes() / 2 ** 20:.0f}MiB"
