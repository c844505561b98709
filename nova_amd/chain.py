"""Chained decode step: the append + attention of every layer of one token in one launch.

A model's layers are chained through their outputs: layer ``l``'s query and new K/V token
come from what layer ``l - 1`` wrote. The per-layer decode step (``KVInt8Cache.update_attend``,
one ``nkv_decode_step_t64`` launch per layer, replacing the ``update`` + ``attend`` pair that
``LeanAttention.forward`` issues for every layer, src/nova/layers.py:132-136) pays one launch's
ramp-up, drain and merge per layer. :class:`ChainedStep` runs the same per-layer computation
for all layers in one launch (``nkv_decode_layers_t64`` / ``_tok``); the int8 prefix of layer
``l + 1``, which does not depend on layer ``l``, streams into on-chip memory while layer ``l``
is merged. Cache state and scalars are bit-identical to the per-layer launches; outputs agree
up to float summation order.

When layer ``l``'s inputs are read (``dep``):

- ``"all"`` (the default): only after every KV head of layer ``l - 1`` has finished, as in a
  model, where every query head of layer ``l`` depends on every head of layer ``l - 1``.
- ``"head"``: an input that is a view of the rows of layer ``l - 1``'s output that its own KV
  head wrote (``q`` the whole output; head ``h``'s k/v rows among its own query heads) is read
  as soon as that head has written it, so each KV head's layers chain on their own. Other
  inputs still wait for every head.

Inputs that neither wait orders (a row of another head's output of the same layer, or, with
``"head"``, of a later layer) are refused when the object is built.

    chain = ChainedStep(cache, keys, values, queries, outs)   # outside graph capture
    chain()                                                   # one step (capturable)
    cache.pos.add_(1)
    chain.check()                                             # outside the loop: raises if a wait gave up

The table of per-layer pointers is built once, on the host and in device memory, so the
tensors passed in must stay allocated (the object keeps references to them) and a captured
graph that launches the chain stays valid while the object lives. The launch assumes every
workgroup of its grid is resident at once; another kernel or process holding CUs can make a
wait give up (after 0.2 s): the affected outputs are then NaN and :meth:`check` raises.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib

D = 128


def _flat_ptr(x: torch.Tensor, name: str, shape: tuple, dtype: torch.dtype, device) -> int:
    if tuple(x.shape) != shape or x.dtype != dtype or x.device != device:
        raise ValueError(f"{name} must be {dtype} {list(shape)} on {device}, got {x.dtype} {list(x.shape)} on {x.device}")
    if not x.is_contiguous() or x.data_ptr() % 16:
        raise ValueError(f"{name} must be contiguous and 16-byte aligned")
    return x.data_ptr()


class ChainedStep:
    """One decode token through ``len(queries)`` layers of ``cache`` (layer ``i`` of the list is
    layer ``i`` of the cache) in one launch.

    keys / values: per layer ``[1, H_kv, 1, 128]`` fp16 (rows contiguous and 16-byte aligned, one
    head stride shared by every layer; views into another layer's output are fine); queries /
    outs: per layer ``[1, H_q, 1, 128]`` contiguous fp16; lses: per layer ``[1, H_q]`` fp32, or
    None. ``cache`` is a :class:`~nova_amd.kvattn.KVInt8Cache` (int8t64) or a
    :class:`~nova_amd.kvtok.KVInt8TokCache` (per-token symmetric). ``n_parts`` is the number of
    streaming workgroups per KV head (0: the library's default for this device). ``dep``:
    ``"all"`` or ``"head"``, when each layer's inputs are read (see the module docstring).
    """

    DEPS = {"head": _lib.NKV_DEP_HEAD, "all": _lib.NKV_DEP_ALL}

    def __init__(self, cache, keys, values, queries, outs, lses=None, n_parts: int = 0, dep: str = "all"):
        from .kvtok import KVInt8TokCache

        lib = _lib.load()
        if dep not in self.DEPS:
            raise ValueError(f"dep must be one of {sorted(self.DEPS)}, got {dep!r}")
        self.dep = dep
        self.cache = cache
        self.tok = isinstance(cache, KVInt8TokCache)
        if getattr(cache, "prefilling", False) or getattr(cache, "_in_prefill", False):
            raise RuntimeError("the chained step decodes one token; finish the prefill first")
        n = len(queries)
        if not (len(keys) == len(values) == len(outs) == n) or (lses is not None and len(lses) != n):
            raise ValueError("keys, values, queries, outs (and lses) need one entry per layer")
        if n < 1 or n > cache.num_slots:
            raise ValueError(f"{n} layers: the cache holds {cache.num_slots}")
        hq, hkv, dev = cache.num_q_heads, cache.num_kv_heads, cache.pos.device
        stride = None
        rows = []
        for i in range(n):
            k, v = keys[i], values[i]
            for name, t in (("key", k), ("value", v)):
                if tuple(t.shape) != (1, hkv, 1, D) or t.dtype != torch.float16 or t.device != dev:
                    raise ValueError(f"{name}[{i}] must be float16 [1, {hkv}, 1, {D}] on {dev}")
                if t.stride(3) != 1 or t.stride(1) % 8 or t.data_ptr() % 16:
                    raise ValueError(f"{name}[{i}] rows must be contiguous and 16-byte aligned")
                if stride is None:
                    stride = t.stride(1)
                elif t.stride(1) != stride:
                    raise ValueError("every key and value must share one head stride")
            q = _flat_ptr(queries[i], f"queries[{i}]", (1, hq, 1, D), torch.float16, dev)
            o = _flat_ptr(outs[i], f"outs[{i}]", (1, hq, 1, D), torch.float16, dev)
            lse = 0
            if lses is not None:
                lse = _flat_ptr(lses[i], f"lses[{i}]", (1, hq), torch.float32, dev)
            if self.tok:
                rows.append([q, k.data_ptr(), v.data_ptr(), cache.kq[i].data_ptr(), cache.ksc[i].data_ptr(),
                             cache.vq[i].data_ptr(), cache.vsc[i].data_ptr(), o, lse])
            else:
                rows.append([q, k.data_ptr(), v.data_ptr(), cache.kq[i].data_ptr(), cache.kmn[i].data_ptr(),
                             cache.kst[i].data_ptr(), cache.vq[i].data_ptr(), cache.vmn[i].data_ptr(),
                             cache.vst[i].data_ptr(), cache.tail_k[i].data_ptr(), cache.tail_v[i].data_ptr(), o, lse])
        # nkv_layer_t64 / nkv_layer_tok: structs of 8-byte pointers, so an int64 array of rows
        self._host = np.ascontiguousarray(np.array(rows, dtype=np.uint64).view(np.int64))
        self._dev = torch.from_numpy(self._host.copy()).to(dev)
        self._keep = (list(keys), list(values), list(queries), list(outs), list(lses or []))
        self.n_layers, self.kv_head_stride = n, int(stride)
        # (the default also caches the device's occupancy, so no query runs under a later capture)
        default = int(lib.nkv_layers_default_parts(hkv, cache.max_len, int(self.tok)))
        parts = int(n_parts) or default
        if parts <= 0:
            raise NotImplementedError("this device cannot hold the chained step's workgroups at once")
        self.n_parts = parts
        self.ws_bytes = int(lib.nkv_layers_workspace_bytes(hkv, hq, parts, n))
        self.workspace = torch.zeros(-(-self.ws_bytes // 4), dtype=torch.int32, device=dev)
        self.ws_bytes = self.workspace.numel() * 4
        self._check_inputs()

    def _check_inputs(self) -> None:
        """Refuse inputs the launch's waits do not order: the library's check of the host table
        (``nkv_decode_layers_check_*``, host only), once here rather than at every launch."""
        _lib.call("nkv_decode_layers_check_tok" if self.tok else "nkv_decode_layers_check_t64", self._host.ctypes.data,
                  self.n_layers, self.kv_head_stride, self.cache.num_q_heads, self.cache.num_kv_heads,
                  self.DEPS[self.dep])

    def _args(self) -> tuple:
        c = self.cache
        head = (self._dev.data_ptr(), self._host.ctypes.data, self.n_layers, self.kv_head_stride)
        tail = (self.workspace.data_ptr(), self.ws_bytes, self.n_parts, self.DEPS[self.dep],
                _lib.stream_ptr(c.pos.device))
        if self.tok:
            return (*head, c.pos.data_ptr(), c._written.data_ptr(), c.num_q_heads, c.num_kv_heads, c.head_dim,
                    c.max_len, *tail)
        return (*head, c.pos.data_ptr(), c.first.data_ptr(), c._written.data_ptr(), c._qlen.data_ptr(),
                c._pg.data_ptr(), c.num_q_heads, c.num_kv_heads, c.head_dim, c.max_len, *tail)

    def __call__(self) -> None:
        """Launch the step on the current stream (capturable: no allocation, no host sync)."""
        _lib.call("nkv_decode_layers_tok" if self.tok else "nkv_decode_layers_t64", *self._args())

    def _sync_words(self) -> list:
        """The sync words at the workspace's end, from the last: the layer counters, the exit
        ticket, the error word, the launch counter (synchronizes)."""
        end = (self.ws_bytes & ~3) // 4
        n = self.n_layers
        return self.workspace[end - n - 3:end].flip(0).tolist()

    def gave_up(self) -> bool:
        """Whether a launch's wait ever gave up (its outputs are then NaN). Synchronizes."""
        return self._sync_words()[self.n_layers + 1] != 0

    def check(self) -> None:
        """Raise ``RuntimeError`` if any launch so far had a wait give up (its outputs are NaN:
        some workgroups were not resident with the others, e.g. another kernel or process held
        CUs). One 4-byte read; synchronizes, so call it outside timed or captured loops."""
        end = (self.ws_bytes & ~3) // 4
        if int(self.workspace[end - self.n_layers - 2].item()) != 0:
            raise RuntimeError("ChainedStep: a chained launch's wait gave up (outputs NaN); every workgroup of "
                               "its grid must be resident at once, so nothing else may hold the GPU's CUs")

    def idle_state(self) -> dict:
        """Between launches: whether layer 0's partial block (the one the next launch polls first;
        each later layer's block is set back to zero by its merger before that layer is published)
        and the counters are back at zero, and the number of launches so far (the forwarding tags'
        counter). Synchronizes."""
        c = self.cache
        part_words = c.num_kv_heads * self.n_parts * (c.num_q_heads // c.num_kv_heads * 128 +
                                                      ((2 * (c.num_q_heads // c.num_kv_heads) + 3) & ~3))
        w = self._sync_words()
        n = self.n_layers
        return {"partials_zero": bool(int(self.workspace[:part_words].abs().sum().item()) == 0),
                "counters_zero": all(x == 0 for x in w[:n + 1]), "error": w[n + 1], "launches": w[n + 2]}
