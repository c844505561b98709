"""The decode step on the library's own scratch array (``nkv_decode_step_static_t64``, no
workspace argument, nothing allocated) against the workspace entry point
(``nkv_decode_step_t64``) through the C ABI.

Both run the same kernels with the same number of parts, so the cache state, the scalars,
the output and the log-sum-exp agree bit for bit. Two configurations run in a row on the
one scratch array, the second smaller (fewer heads, fewer parts, shorter context), then the
first again: the publication area each call leaves cleared is what the next one starts from.
"""

from __future__ import annotations

import pytest
import torch

from tests.helpers import D, make

pytestmark = pytest.mark.gpu

STATE = ("kq", "vq", "kmn", "kst", "vmn", "vst", "tail_k", "tail_v")
SCALARS = ("_written", "_qlen", "_pg")


class _Pair:
    """Two caches with the same prefill: ``ws`` steps through ``nkv_decode_step_t64``,
    ``st`` through ``nkv_decode_step_static_t64``."""

    def __init__(self, hq: int, hkv: int, max_len: int, used0: int, steps: int, seed: int):
        from nova_amd.kvattn import KVInt8Cache

        q, k, v = make(used0 + steps, seed=seed, hq=hq, hkv=hkv)
        self.q, self.k, self.v = q.cuda(), k.cuda(), v.cuda()
        self.ws, self.st = (KVInt8Cache(num_slots=1, num_kv_heads=hkv, head_dim=D, max_len=max_len, num_q_heads=hq)
                            for _ in range(2))
        for c in (self.ws, self.st):
            c.begin_prefill(used0)
            c.set_prefill_pos(0)
            c.update(self.k[:, :, :used0], self.v[:, :, :used0], 0)
            c.finish_prefill(used0)
        self.p = used0

    def step(self, tag: str) -> None:
        from nova_amd import _lib

        p = self.p
        print(f"case {tag} pos={p}", flush=True)
        kn, vn = self.k[:, :, p:p + 1], self.v[:, :, p:p + 1]
        for c in (self.ws, self.st):
            c.pos.fill_(p)
        self.ws.update_attend(kn, vn, self.q, 0)
        args = self.st.step_args(kn, vn, self.q, 0)
        assert args[23] == self.st._ws.data_ptr()  # workspace, workspace_bytes: not passed
        _lib.call("nkv_decode_step_static_t64", *args[:23], *args[25:])
        torch.cuda.synchronize()
        for nm in STATE:
            assert torch.equal(getattr(self.ws, nm)[0], getattr(self.st, nm)[0]), (tag, p, nm)
        for nm in SCALARS:
            assert torch.equal(getattr(self.ws, nm), getattr(self.st, nm)), (tag, p, nm)
        assert torch.equal(self.ws.merged, self.st.merged), (tag, p)
        assert torch.equal(self.ws.lse, self.st.lse), (tag, p)
        self.p += 1


def test_static_scratch_step_equals_workspace_step():
    # 32K-token context at 32 query / 8 KV heads (32 parts per head), then 8 / 2 heads over
    # a 512-token cache (1 part per head) across two group boundaries, then the first again
    big = _Pair(hq=32, hkv=8, max_len=32768 + 128, used0=32700, steps=6, seed=71)
    small = _Pair(hq=8, hkv=2, max_len=512, used0=250, steps=80, seed=72)
    assert big.st._n_parts == 32 and small.st._n_parts == 1
    for _ in range(3):
        big.step("32k hq32 hkv8")
    for _ in range(80):
        small.step("512 hq8 hkv2")
    for _ in range(3):
        big.step("32k hq32 hkv8 again")


def test_static_scratch_rejects_calls_beyond_its_size():
    """More partial bytes than the array holds: an error before anything is launched."""
    from nova_amd import _lib

    lib = _lib.load()
    fake = 1 << 20  # never dereferenced: the size check returns first
    args = [fake] * 3 + [128] + [fake] * 13 + [128, 8, 128, 1 << 16, fake, fake, 64, None]
    rc = lib.nkv_decode_step_static_t64(*args)
    assert rc == _lib.NKV_ERR_UNSUPPORTED
    assert b"static scratch" in lib.nkv_last_error()
