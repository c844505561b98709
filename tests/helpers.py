"""Shared helpers of the GPU parity tests: seeded CPU inputs, fp16 ULP distance, criteria."""

from __future__ import annotations

import numpy as np
import torch

HQ, H_KV, D = 32, 8, 128
FP16_TINY = float(np.finfo(np.float16).tiny)


def randn(shape, seed: int, scale: float = 0.7) -> torch.Tensor:
    """Seeded N(0, scale^2) fp16 tensor generated on the CPU (reproducible anywhere)."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.float16)


def make(used: int, seed: int = 0, outliers: bool = False, hq: int = HQ, hkv: int = H_KV):
    """q, k, v like ``tests/test_kvattn.py:48-59``: N(0, 0.49) fp16; ``outliers`` scales
    channels 3, 71, 120 of K by 65."""
    k = randn((1, hkv, used, D), seed)
    if outliers:
        s = torch.ones(D)
        s[torch.tensor([3, 71, 120])] = 65.0
        k = (k.float() * s).to(torch.float16)
    v = randn((1, hkv, used, D), seed + 1000)
    q = randn((1, hq, 1, D), seed + 2000)
    return q, k, v


def bench_outliers(k: torch.Tensor, seed: int, n_ch: int = 4, gain: float = 8.0) -> torch.Tensor:
    """4 seeded random K channels per head scaled x8 (the long-context workload's K)."""
    g = torch.Generator().manual_seed(seed)
    k = k.clone()
    for h in range(k.shape[1]):
        ch = torch.randperm(k.shape[-1], generator=g)[:n_ch]
        k[:, h, :, ch] = (k[:, h, :, ch].float() * gain).to(torch.float16)
    return k


def ulp(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Element-wise distance in units of the fp16 spacing at ``want`` (``tests/test_kvattn.py:73-77``)."""
    want16 = want.astype(np.float16)
    up = np.abs(np.nextafter(want16, np.float16(np.inf)).astype(np.float64) - want16.astype(np.float64))
    up = np.maximum(up, FP16_TINY * 2.0 ** -10)
    return np.abs(got.astype(np.float64) - want16.astype(np.float64)) / up


def assert_ulp_or_abs(got, want, max_ulp: float, abs_tol: float, tag: str = "") -> dict:
    """Every element within ``max_ulp`` fp16 ULP or ``abs_tol`` absolute of ``want``; every
    element of ``got`` and ``want`` finite (a NaN fails the comparisons, so it is checked first)."""
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want)
    assert np.isfinite(got).all(), f"{tag}: {int((~np.isfinite(got)).sum())} non-finite outputs"
    assert np.isfinite(want.astype(np.float64)).all(), f"{tag}: non-finite reference values"
    u = ulp(got, want)
    diff = np.abs(got.astype(np.float64) - want.astype(np.float16).astype(np.float64))
    bad = (u > max_ulp) & (diff > abs_tol)
    assert int(bad.sum()) == 0, (f"{tag}: {int(bad.sum())} elements beyond {max_ulp} ULP and {abs_tol:g} abs "
                                 f"(max ULP {u.max():.2f}, max abs {diff.max():.2e})")
    return {"max_ulp": float(u.max()), "max_abs": float(diff.max()),
            "exact": float((got.astype(np.float16) == want.astype(np.float16)).mean())}


def npy(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()
