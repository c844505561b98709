"""ctypes binding of ``libnova_kv.so`` (the C ABI declared in ``include/nova_kv.h``).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7`` dependency
resolves to the HIP runtime torch already mapped (same soname): device pointers
and ``hipStream_t`` handles from torch are then valid inside the library.

There is no fallback: if the library is missing, or the process has no GPU, the
calls raise ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libnova_kv.so"

NKV_OK = 0
NKV_ERR_INVALID = 1
NKV_ERR_UNSUPPORTED = 2
NKV_ERR_HIP = 3

NKV_F16, NKV_BF16, NKV_F32 = 0, 1, 2
NKV_AXIS_CHANNEL, NKV_AXIS_TOKEN = 0, 1
NKV_DEP_HEAD, NKV_DEP_ALL = 0, 1

P = c_void_p
I64 = c_int64
I32 = c_int

# name -> (restype, argtypes); must match include/nova_kv.h
# q, k_new, v_new, kv_head_stride, kq, kmn, kst, vq, vmn, vst, tail_k, tail_v, pos, first, written,
# qlen, pg, hq, hkv, head_dim, capacity, out, lse, workspace, workspace_bytes, n_parts, stream
_STEP = [P, P, P, I64, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, P, P, P, I64, I64, P]
# the same without workspace and workspace_bytes
_STEP_STATIC = _STEP[:23] + _STEP[25:]
# q, k_new, v_new, kv_head_stride, kq, ksc, vq, vsc, pos, written, hq, hkv, head_dim, capacity, out,
# lse, workspace, workspace_bytes, n_parts, stream
_STEP_TOK = [P, P, P, I64, P, P, P, P, P, P, I64, I64, I64, I64, P, P, P, I64, I64, P]

SIGNATURES = {
    "nkv_abi_version": (c_int, []),
    "nkv_last_error": (ctypes.c_char_p, []),
    "nkv_quantize_int8": (c_int, [P, c_int, I64, I64, I64, I64, I64, c_int, P, I64, P, P, I64, P]),
    "nkv_dequantize_int8": (c_int, [P, I64, P, P, I64, I64, I64, I64, I64, c_int, P, c_int, I64, P]),
    "nkv_attn_decode_t64": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, P, P, P, P, P, P,
                                    P, P, P, I64, I64, P]),
    "nkv_attn_workspace_bytes": (I64, [I64, I64, I64]),
    "nkv_attn_default_parts": (I64, [I64, I64]),
    "nkv_append_t64": (c_int, [P, P, I64, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, P]),
    "nkv_decode_step_t64": (c_int, _STEP),
    "nkv_decode_step_partials_t64": (c_int, _STEP),
    "nkv_decode_step_combine_t64": (c_int, _STEP),
    "nkv_decode_step_static_t64": (c_int, _STEP_STATIC),
    "nkv_tail_attend": (c_int, [P, P, P, P, I64, I64, I64, I64, P, P, P]),
    "nkv_ring_mask": (c_int, [P, P, P, I64, P, P]),
    "nkv_quantize_tok": (c_int, [P, c_int, I64, I64, I64, I64, P, I64, P, I64, P]),
    "nkv_dequantize_tok": (c_int, [P, I64, P, I64, I64, I64, I64, P, c_int, I64, P]),
    "nkv_attn_decode_tok": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, P, P, P, P, I64, I64, P]),
    "nkv_append_tok": (c_int, [P, P, I64, P, P, P, P, P, P, I64, I64, I64, P]),
    "nkv_decode_step_tok": (c_int, _STEP_TOK),
    "nkv_decode_step_partials_tok": (c_int, _STEP_TOK),
    "nkv_decode_step_combine_tok": (c_int, _STEP_TOK),
    "nkv_layers_workspace_bytes": (I64, [I64, I64, I64, I64]),
    "nkv_layers_default_parts": (I64, [I64, I64, c_int]),
    # layers_dev, layers_host, n_layers, kv_head_stride, pos, first, written, qlen, pg, hq, hkv, head_dim,
    # capacity, workspace, workspace_bytes, n_parts, stream
    "nkv_decode_layers_t64": (c_int, [P, P, I64, I64, P, P, P, P, P, I64, I64, I64, I64, P, I64, I64, I32, P]),
    # layers_dev, layers_host, n_layers, kv_head_stride, pos, written, hq, hkv, head_dim, capacity,
    # workspace, workspace_bytes, n_parts, stream
    "nkv_decode_layers_tok": (c_int, [P, P, I64, I64, P, P, I64, I64, I64, I64, P, I64, I64, I32, P]),
    "nkv_decode_layers_check_t64": (c_int, [P, I64, I64, I64, I64, I32]),
    "nkv_decode_layers_check_tok": (c_int, [P, I64, I64, I64, I64, I32]),
    "nkv_paged_workspace_bytes": (I64, [I64, I64, I64]),
    "nkv_paged_quantize_t64": (c_int, [P, c_int, I64, I64, I64, c_int, P, P, I64, I64, P]),
    "nkv_paged_append_t64": (c_int, [P, P, I64, I64, P, P, I64, I64, P, P, I64, I64, I64, P]),
    "nkv_paged_attn_decode_t64": (c_int, [P, P, P, I64, I64, P, P, I64, I64, I64, I64, P, P, I64, P, P, P, I64, P]),
    "nkv_paged_decode_step_t64": (c_int, [P, P, P, I64, I64, P, P, I64, I64, P, P, I64, I64, I64, I64, P, P, I64, P,
                                          P, P, I64, P]),
    "nkv_paged_quantize_tok": (c_int, [P, c_int, I64, I64, I64, c_int, P, P, I64, I64, P]),
    "nkv_paged_decode_step_tok": (c_int, [P, P, P, I64, I64, P, P, I64, I64, P, I64, I64, I64, I64, P, P, I64, P,
                                          P, P, I64, P]),
    "nkv_prefill_workspace_bytes": (I64, [I64, I64, I64, I64]),
    "nkv_prefill_default_splits": (I64, [I64, I64, I64, I64]),
    "nkv_prefill_attn_t64": (c_int, [P, P, P, I64, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, I64, I64, P]),
    "nkv_prefill_attn_hist_t64": (c_int, [P, I64, P, P, I64, I64, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P,
                                          I64, I64, P]),
    "nkv_copy_bytes": (c_int, [P, P, I64, P]),
    "nkv_read_bw": (c_int, [P, I64, P, I64, P]),
    "nkv_clock_probe": (c_int, [P, I64, I64, P]),
    "nkv_read_bw_lds": (c_int, [P, I64, P, I64, P]),
    "nkv_l2_handover": (c_int, [c_int, P, P]),
    "nkv_decode_step_qkv_workspace_bytes": (I64, [I64, I64, I64, I64]),
    # x, x_gamma, x_eps, w_qkv, hidden, q_gamma, k_gamma, qk_eps, inv_freq, qkv_out, kq, kmn, kst, vq, vmn,
    # vst, tail_k, tail_v, pos, first, written, qlen, pg, hq, hkv, head_dim, capacity, out, lse, w_o,
    # h1_out, workspace, workspace_bytes, n_parts, stream
    "nkv_decode_step_qkv_t64": (c_int, [P, P, c_float, P, I64, P, P, c_float, P, P, P, P, P, P, P, P, P, P, P, P, P,
                                        P, P, I64, I64, I64, I64, P, P, P, P, P, I64, I64, P]),
    "nkv_gemv": (c_int, [P, P, c_float, P, I64, I64, P, P, P]),
    "nkv_swiglu_gemv": (c_int, [P, P, c_float, P, I64, I64, P, P]),
    "nkv_qk_norm_rope": (c_int, [P, I64, I64, I64, P, P, c_float, P, P, P]),
}

ABI_VERSION = 11

_lib = None
_lock = threading.Lock()
_l2_probed = False


class NovaKVError(RuntimeError):
    """A failing ``nkv_*`` call; ``code`` is the NKV_ERR_* status."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def load(require_gpu: bool = True):
    """Load (once) and return the ctypes handle of ``libnova_kv.so``."""
    global _lib
    if require_gpu and not torch.cuda.is_available():
        raise RuntimeError("nova_amd needs a ROCm GPU (gfx950); none is visible to torch")
    if _lib is not None:
        if not _l2_probed and require_gpu:
            _probe_l2()
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m nova_amd.build`")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.nkv_abi_version() != ABI_VERSION:
                raise RuntimeError(f"libnova_kv ABI {lib.nkv_abi_version()} != {ABI_VERSION}: rebuild it")
            _lib = lib
    if require_gpu:
        _probe_l2()
    return _lib


def _probe_l2() -> None:
    """Turn on the XCD-local hand-over for the current device (``nkv_l2_handover``), unless
    ``NKV_L2_HANDOVER=0``. The probe synchronizes, so under stream capture it waits for the
    next call outside capture."""
    global _l2_probed
    if torch.cuda.is_current_stream_capturing():
        return
    with _lock:
        if _l2_probed:
            return
        _l2_probed = True
    l2_handover(os.environ.get("NKV_L2_HANDOVER", "1") != "0")


def l2_handover(enable: bool = True) -> int:
    """Probe the current device and turn the XCD-local hand-over on (``enable``) or off; returns
    the XCD count it runs with (0: off). Call outside stream capture."""
    n = ctypes.c_int64(0)
    call("nkv_l2_handover", 1 if enable else 0, ctypes.byref(n), stream_ptr())
    return int(n.value)


def call(name: str, *args) -> None:
    """Call ``name``; raise ``ValueError`` (invalid argument), ``NotImplementedError``
    (unsupported here) or ``NovaKVError`` (HIP failure) on a nonzero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != NKV_OK:
        msg = lib.nkv_last_error().decode("utf-8", "replace")
        if rc == NKV_ERR_INVALID:
            raise ValueError(f"{name}: {msg}")
        if rc == NKV_ERR_UNSUPPORTED:
            raise NotImplementedError(f"{name}: {msg}")
        raise NovaKVError(rc, f"{name}: {msg}")


def stream_ptr(device: torch.device | None = None) -> int:
    """The current torch stream of ``device`` as a raw ``hipStream_t``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_WORKSPACES: dict[str, torch.Tensor] = {}
# Workspaces replaced by larger ones. A graph captured earlier may still hold a raw pointer
# into one, so they stay allocated for the life of the process.
_RETIRED: list[torch.Tensor] = []


def workspace(device: torch.device, nbytes: int, kind: str = "scratch") -> torch.Tensor:
    """A cached per-device, zero-filled byte workspace of at least ``nbytes``. It grows only
    outside graph capture (a capture that needs more raises); the buffer it replaces is kept,
    never freed, because a captured graph may point into it. Callers pass the whole buffer
    (``numel()`` bytes)."""
    key = f"{device}/{kind}"
    w = _WORKSPACES.get(key)
    if w is None or w.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"workspace '{kind}' must grow to {nbytes} bytes inside a graph capture; "
                               "pass a preallocated scratch buffer")
        if w is not None:
            _RETIRED.append(w)
        w = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = w
    return w
