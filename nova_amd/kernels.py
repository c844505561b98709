"""Availability gate of the HIP kernels — counterpart of ``triton_available()``
(src/nova/kernels.py:75-94), which the reference's GPU tests use as their skip condition."""

from __future__ import annotations

import torch

_OK: bool | None = None


def hip_available() -> bool:
    """True when a GPU is visible and ``libnova_kv.so`` loads and runs a tiny kernel.

    The probe runs once (a ring-mask launch on fixed device scalars) and is cached.
    """
    global _OK
    if _OK is not None:
        return _OK
    if not torch.cuda.is_available():
        _OK = False
        return False
    try:
        from . import _lib

        _lib.load()
        s = torch.tensor([70, 64, 0], dtype=torch.int64, device="cuda")
        m = torch.empty(64, dtype=torch.uint8, device="cuda")
        _lib.call("nkv_ring_mask", s[0:].data_ptr(), s[1:].data_ptr(), s[2:].data_ptr(), 64, m.data_ptr(),
                  _lib.stream_ptr())
        torch.cuda.synchronize()
        _OK = int(m.sum().item()) == 6
    except Exception:  # noqa: BLE001
        _OK = False
    return _OK


triton_available = hip_available  # the name the reference's tests import
