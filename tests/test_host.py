"""Host-side logic that needs no GPU: capacity buckets, the additive mask row, byte accounting."""

from __future__ import annotations

from types import SimpleNamespace

import torch

from oracle import decode as odec
from oracle import kvquant as okq


def test_bucket_for_boundaries():
    """``tests/test_decode_mask_bucket.py:29-37``."""
    from nova_amd.decode import BUCKETS, bucket_for

    assert BUCKETS == odec.BUCKETS
    for n in (1, 2070, 2071, 8192, 16384 + 64, 32768 + 256, 65536, 70000):
        assert bucket_for(n) == odec.bucket_for(n)
    assert bucket_for(1) == 2070 and bucket_for(2071) == 4096 and bucket_for(70000) == 70000


def test_mask_row_matches_table_bitwise():
    """``_mask_row(pos)`` equals row ``pos`` of ``_build_mask_table`` including the min
    values (``tests/test_decode_mask_bucket.py:40-57``), and the oracle's row."""
    from nova_amd.decode import GraphDecoder

    max_len = 64
    table = GraphDecoder._build_mask_table(max_len, torch.float16, "cpu")
    fake = SimpleNamespace(max_len=max_len, _arange=torch.arange(max_len, dtype=torch.long),
                           _zero=torch.zeros((), dtype=torch.float16),
                           _ninf=torch.full((), torch.finfo(torch.float16).min, dtype=torch.float16))
    for pos in (0, 1, 7, 63):
        row = GraphDecoder._mask_row(fake, torch.tensor([pos]))
        assert row.shape == (1, 1, 1, max_len)
        assert torch.equal(row.reshape(max_len), table[pos])
        assert torch.equal(row.reshape(max_len), torch.from_numpy(odec.mask_row(pos, max_len)))


def test_bytes_per_token_int8():
    from nova_amd.kvquant import bytes_per_token

    a = bytes_per_token(36, 8, 128, bits=8)
    b = bytes_per_token(36, 8, 128, bits=8, k_axis="token", token_group=64)
    assert a == okq.bytes_per_token_int8(36, 8, 128)
    assert b == okq.bytes_per_token_int8(36, 8, 128, k_axis="token", token_group=64)
    assert 1.85 <= b["ratio"] <= 1.95
