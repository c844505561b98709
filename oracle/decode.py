"""numpy restatement of the decoder's capacity buckets and mask row (checker only)."""

from __future__ import annotations

import numpy as np

BUCKETS = (2070, 4096, 8192, 16384, 32768, 65536)  # src/nova/decode.py:39


def bucket_for(n: int, buckets=BUCKETS) -> int:
    """Smallest bucket >= n, else n itself (``src/nova/decode.py:42-48``)."""
    n = int(n)
    for b in buckets:
        if n <= b:
            return int(b)
    return n


def mask_row(pos: int, max_len: int) -> np.ndarray:
    """Additive fp16 mask row: 0 for ``i <= pos``, ``finfo(fp16).min`` elsewhere
    (``src/nova/decode.py:200-205``)."""
    neg = np.finfo(np.float16).min
    return np.where(np.arange(max_len) <= pos, np.float16(0), np.float16(neg)).astype(np.float16)
