"""GPU parity of the MFMA chunked-prefill attention over the int8t64 cache.

Oracle: ``oracle.attn.chunk_prefill_attend`` (fp64; pinned in ``tests/test_oracle.py``).
The kernel rounds the softmax weights to one fp16 operand (scaled by 2^15), as a fused
fp16 attention does, so the bar is the path's output criterion: max-abs <= 2e-3 against
the oracle, plus a tight mean error that a wrong row or mask would break.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from tests.helpers import D, npy, randn

pytestmark = pytest.mark.gpu


def _case(hq, hkv, used, m, seed, cap_extra=64):
    from nova_amd.kvattn import pack_int8_kv

    k = randn((1, hkv, used + cap_extra, D), seed, 1.0)
    v = randn((1, hkv, used + cap_extra, D), seed + 1, 1.0)
    packed = [t.contiguous() for t in pack_int8_kv(k.cuda(), v.cuda())]
    kch = randn((1, hkv, m, D), seed + 2, 1.0).cuda()
    vch = randn((1, hkv, m, D), seed + 3, 1.0).cuda()
    q = randn((1, hq, m, D), seed + 4, 1.0).cuda()
    return q, kch, vch, packed


def _check(got, q, kch, vch, packed, used, heads=None, tag=""):
    kq, kmn, kst, vq, vmn, vst = (npy(t)[0] for t in packed)
    want = oattn.chunk_prefill_attend(npy(q)[0], kq, kmn, kst, vq, vmn, vst, used, npy(kch)[0], npy(vch)[0], heads)
    g = npy(got)[0].astype(np.float64)
    if heads is not None:
        gq = q.shape[1] // kch.shape[1]
        rows = [h * gq + j for h in heads for j in range(gq)]
        g, want = g[rows], want[rows]
    err = np.abs(g - want)
    assert err.max() <= 2e-3, f"{tag}: max abs {err.max():.2e}"
    assert err.mean() <= 1.5e-4, f"{tag}: mean abs {err.mean():.2e}"
    return err


@pytest.mark.parametrize("used,m", [(0, 1), (0, 70), (64, 1), (64, 65), (512, 17), (512, 130), (2048, 256)])
def test_prefill_against_oracle(used, m):
    from nova_amd.kvattn import int8_prefill_attend

    print(f"case used={used} m={m}", flush=True)
    q, kch, vch, packed = _case(32, 8, used, m, seed=60 + m)
    got = int8_prefill_attend(q, kch, vch, *packed, used=used)
    _check(got, q, kch, vch, packed, used, tag=f"used={used} m={m}")


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 2)])
def test_prefill_gqa_ratios(hq, hkv):
    from nova_amd.kvattn import int8_prefill_attend

    q, kch, vch, packed = _case(hq, hkv, 256, 90, seed=70 + hq)
    got = int8_prefill_attend(q, kch, vch, *packed, used=256)
    _check(got, q, kch, vch, packed, 256, tag=f"hq={hq} hkv={hkv}")


def test_prefill_split_settings_agree():
    from nova_amd.kvattn import int8_prefill_attend

    q, kch, vch, packed = _case(32, 8, 1024, 100, seed=80)
    outs = [int8_prefill_attend(q, kch, vch, *packed, used=1024, splits=s).clone() for s in (1, 2, 5)]
    for o in outs:
        _check(o, q, kch, vch, packed, 1024, tag="splits")
    assert (outs[0].float() - outs[1].float()).abs().max().item() <= 1e-3


@pytest.mark.parametrize("used,splits", [(128, 1), (192, 1), (256, 2)])
def test_prefill_few_groups_per_split(used, splits):
    """Splits of two and three cache groups: the loop's start (two stages loaded before the first
    group) and its end (no further load; the last group dequantizes a stale stage into a tile
    buffer nothing reads) meet within a few groups."""
    from nova_amd.kvattn import int8_prefill_attend

    print(f"case used={used} splits={splits}", flush=True)
    q, kch, vch, packed = _case(32, 8, used, 40, seed=90 + used)
    got = int8_prefill_attend(q, kch, vch, *packed, used=used, splits=splits)
    _check(got, q, kch, vch, packed, used, tag=f"used={used} splits={splits}")


def test_prefill_chunk_512_over_16k():
    """The chunked-prefill workload: a 512-token chunk over a 16384-token int8 cache, 32 q /
    8 KV heads; checked on KV heads 0 and 7 (the fp64 oracle over all heads is slow)."""
    from nova_amd.kvattn import int8_prefill_attend

    q, kch, vch, packed = _case(32, 8, 16384, 512, seed=90, cap_extra=0)
    got = int8_prefill_attend(q, kch, vch, *packed, used=16384)
    assert torch.isfinite(got).all()
    _check(got, q, kch, vch, packed, 16384, heads=[0, 7], tag="16k")


@pytest.mark.parametrize("profile", ["jump", "rise"])
def test_prefill_scores_that_move_the_softmax_reference(profile):
    """As the decode test of the same name: cache scores with a late large jump, or rising over
    the whole cache, against the oracle at the prefill criterion."""
    from nova_amd.kvattn import int8_prefill_attend, pack_int8_kv

    used, m = 2048, 65
    q, kch, vch, _ = _case(32, 8, used, m, seed=81)
    k = randn((1, 8, used + 64, D), 81, 1.0)
    v = randn((1, 8, used + 64, D), 82, 1.0)
    kf, qf = k.float(), q.float().cpu()[0, :, 0]
    for h in range(8):
        dirv = qf[4 * h] / qf[4 * h].norm()
        if profile == "jump":
            kf[0, h, used - 300] += 40.0 * dirv
        else:
            kf[0, h, :used] += torch.linspace(0.0, 20.0, used)[:, None] * dirv[None, :]
    packed = [t.contiguous() for t in pack_int8_kv(kf.half().cuda(), v.cuda())]
    got = int8_prefill_attend(q, kch, vch, *packed, used=used)
    _check(got, q, kch, vch, packed, used, tag=profile)


@pytest.mark.parametrize("used,n", [(0, 64), (0, 130), (512, 64), (512, 130)])
def test_prefill_with_fp16_history(used, n):
    """The fp16-history branch (``m > n``: a staged prefill's later chunks attend the earlier
    ones in fp16): 192 history tokens before the chunk, after ``used`` int8 tokens."""
    from nova_amd.kvattn import int8_prefill_attend

    hist = 192
    print(f"case history used={used} hist={hist} n={n}", flush=True)
    q, kch, vch, packed = _case(32, 8, used, hist + n, seed=100 + used + n)
    q = q[:, :, hist:].contiguous()
    got = int8_prefill_attend(q, kch, vch, *packed, used=used)
    _check(got, q, kch, vch, packed, used, tag=f"history used={used} n={n}")


def test_staged_prefill_in_three_chunks_against_oracle():
    """``KVInt8Cache`` staged prefill in three chunks of 100, 130 and 70 tokens over two layers:
    every chunk's ``attend_prefill`` output (chunks 2 and 3 read the earlier chunks from the fp16
    staging area) against the oracle's causal attention over the fp16 tokens up to it."""
    from nova_amd.kvattn import KVInt8Cache

    print("case staged prefill 3 chunks", flush=True)
    L, hq, hkv, total, chunks = 2, 32, 8, 300, (100, 130, 70)
    cache = KVInt8Cache(num_slots=L, num_kv_heads=hkv, head_dim=D, max_len=512, num_q_heads=hq)
    ks = [randn((1, hkv, total, D), 110 + l, 1.0) for l in range(L)]
    vs = [randn((1, hkv, total, D), 120 + l, 1.0) for l in range(L)]
    qs = [randn((1, hq, total, D), 130 + l, 1.0) for l in range(L)]
    none8 = np.zeros((hkv, 64, D), np.uint8)
    none16 = np.zeros((hkv, 1, D), np.float16)
    cache.begin_prefill(total)
    off = 0
    for n in chunks:
        cache.set_prefill_pos(off)
        for l in range(L):
            cache.update(ks[l][:, :, off:off + n].cuda(), vs[l][:, :, off:off + n].cuda(), l)
            got = npy(cache.attend_prefill(qs[l][:, :, off:off + n].cuda(), l))[0].astype(np.float64)
            want = oattn.chunk_prefill_attend(npy(qs[l])[0, :, off:off + n], none8, none16, none16, none8, none16,
                                              none16, 0, npy(ks[l])[0, :, :off + n], npy(vs[l])[0, :, :off + n])
            err = np.abs(got - want)
            assert err.max() <= 2e-3 and err.mean() <= 1.5e-4, (f"chunk at {off} layer {l}: max {err.max():.2e} "
                                                                 f"mean {err.mean():.2e}")
        off += n
    cache.finish_prefill(total)
