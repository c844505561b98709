"""fp16 static KV cache — the prefill staging area of the int8 cache.

Mirrors ``StaticKVCache`` (src/nova/cache.py:117-175): per-layer
``[batch, H_kv, max_len, D]`` fp16 buffers, a device write cursor ``pos``, in-place
``index_copy_`` for one decode token and a slice write for a prefill chunk.
"""

from __future__ import annotations

import torch


class StaticKVCache:
    """``update()`` has the signature of an HF ``Cache.update``."""

    def __init__(self, num_slots: int, num_kv_heads: int, head_dim: int, max_len: int, batch: int = 1,
                 dtype: torch.dtype = torch.float16, device: str | torch.device = "cuda") -> None:
        self.num_slots = num_slots
        self.max_len = max_len
        self.batch = batch
        self.dtype = dtype
        self.device = device
        shape = (batch, num_kv_heads, max_len, head_dim)
        self.key_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_slots)]
        self.value_cache = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_slots)]
        self.pos = torch.zeros(1, dtype=torch.long, device=device)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self.pos.item())

    def reset(self) -> None:
        self.pos.zero_()

    def update(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int):
        """One decode token written at ``pos`` in place (graph-safe); a chunk goes to
        :meth:`append_prefill`. Returns the whole layer cache."""
        if key.shape[2] != 1:
            return self.append_prefill(key, value, layer_idx)
        self.key_cache[layer_idx].index_copy_(2, self.pos, key)
        self.value_cache[layer_idx].index_copy_(2, self.pos, value)
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def append_prefill(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int):
        """Write ``n`` positions starting at ``pos`` (eager only: reads ``pos`` on the host)."""
        n = key.shape[2]
        start = int(self.pos.item())
        self.key_cache[layer_idx][:, :, start:start + n] = key
        self.value_cache[layer_idx][:, :, start:start + n] = value
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.key_cache + self.value_cache)
