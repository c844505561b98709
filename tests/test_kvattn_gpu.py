"""GPU parity of the fused int8 decode attention — restates the reference's
``tests/test_kvattn.py`` against the HIP kernel.

Oracle: dequantize with the stored fp16 rulers, then softmax attention in fp64
(``oracle.attn.int8_attn_decode``; the reference uses torch's fp32 math SDPA, which
``tests/test_oracle.py`` pins to the same values). Criterion, as the reference's
(``tests/test_kvattn.py:80-93``): every element within 2 fp16 ULP or 1e-5 absolute.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from tests.helpers import D, H_KV, HQ, assert_ulp_or_abs, bench_outliers, make, npy, randn

pytestmark = pytest.mark.gpu


def _packed(k, v):
    from nova_amd.kvattn import pack_int8_kv

    return pack_int8_kv(k.cuda(), v.cuda())


def _want(q, packed, used):
    kq, kmn, kst, vq, vmn, vst = (npy(t)[0] for t in packed)
    out, lse = oattn.int8_attn_decode(npy(q)[0, :, 0], kq, kmn, kst, vq, vmn, vst, used)
    return out, lse


@pytest.mark.parametrize("used", [7, 63, 64, 65, 511, 512, 513, 1024, 2049, 4096])
def test_ulp_against_dequant_then_attention(used):
    from nova_amd.kvattn import int8_attn_decode

    print(f"case used={used}", flush=True)
    q, k, v = make(used)
    packed = _packed(k, v)
    want, _ = _want(q, packed, used)
    got = int8_attn_decode(q.cuda(), *packed, used=used)
    st = assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, f"used={used}")
    assert st["max_ulp"] <= 2.0, st
    assert st["exact"] > 0.97, st


@pytest.mark.parametrize("used", [300, 2049])
def test_ulp_under_channel_outliers(used):
    from nova_amd.kvattn import int8_attn_decode

    q, k, v = make(used, seed=1, outliers=True)
    packed = _packed(k, v)
    want, _ = _want(q, packed, used)
    got = int8_attn_decode(q.cuda(), *packed, used=used)
    assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, f"outliers used={used}")


@pytest.mark.parametrize("chunk", [64, 512, 4096])
def test_split_settings_agree(chunk):
    from nova_amd.kvattn import int8_attn_decode

    used = 1024
    q, k, v = make(used, seed=2)
    packed = _packed(k, v)
    want, _ = _want(q, packed, used)
    got = int8_attn_decode(q.cuda(), *packed, used=used, chunk=chunk)
    assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, f"chunk={chunk}")


def test_gqa_head_mapping():
    """Constant V per KV head: Q head h returns KV head h // 4's constant, exactly."""
    from nova_amd.kvattn import int8_attn_decode

    used = 256
    k = randn((1, H_KV, used, D), 3, 1.0)
    v = torch.arange(H_KV, dtype=torch.float16).view(1, H_KV, 1, 1).expand(1, H_KV, used, D).contiguous()
    q = randn((1, HQ, 1, D), 4, 1.0)
    got = int8_attn_decode(q.cuda(), *_packed(k, v), used=used)
    want = torch.arange(HQ, dtype=torch.float16) // (HQ // H_KV)
    assert torch.equal(got[0, :, 0, 0].cpu(), want), got[0, :, 0, 0].tolist()


def test_used_ignores_unwritten_slots():
    """Garbage codes and rulers past ``used`` leave the output bit-identical."""
    from nova_amd.kvattn import GROUP_T, int8_attn_decode

    used, capacity = 300, 640
    q, k, v = make(used, seed=4)
    kq, kmn, kst, vq, vmn, vst = _packed(k, v)
    big = lambda t, fill, n: torch.cat([t, torch.full((1, H_KV, n, D), fill, dtype=t.dtype, device="cuda")], 2)  # noqa: E731
    pad_g = -(-capacity // GROUP_T) - kmn.shape[2]
    args = (big(kq, 255, capacity - used), big(kmn, 300.0, pad_g), big(kst, 9.0, pad_g),
            big(vq, 255, capacity - used), big(vmn, 300.0, pad_g), big(vst, 9.0, pad_g))
    qc = q.cuda()
    want = int8_attn_decode(qc, kq, kmn, kst, vq, vmn, vst, used=used)
    got = int8_attn_decode(qc, *args, used=used)
    assert torch.equal(got, want)


def test_zero_used_returns_zeros():
    from nova_amd.kvattn import int8_attn_decode

    q, k, v = make(64)
    lse = torch.zeros(1, HQ, dtype=torch.float32, device="cuda")
    out = int8_attn_decode(q.cuda(), *_packed(k, v), used=0, lse_out=lse)
    assert torch.equal(out, torch.zeros_like(out))
    assert torch.isneginf(lse).all()


def test_lse_matches_oracle():
    from nova_amd.kvattn import int8_attn_decode

    used = 777
    q, k, v = make(used, seed=9)
    packed = _packed(k, v)
    lse = torch.zeros(1, HQ, dtype=torch.float32, device="cuda")
    int8_attn_decode(q.cuda(), *packed, used=used, lse_out=lse)
    _, want = _want(q, packed, used)
    np.testing.assert_allclose(npy(lse)[0], want, rtol=1e-5, atol=1e-5)


def test_graph_capture_replays_bitwise():
    """Captured into a graph and replayed several times with eager work in between,
    every replay equals the eager result bit for bit (``tests/test_kvattn.py:178-206``)."""
    from nova_amd.kvattn import PAD_M, int8_attn_decode

    used, chunk = 1024, 512
    q, k, v = make(used, seed=6)
    packed = _packed(k, v)
    qc = q.cuda()
    want = int8_attn_decode(qc, *packed, used=used, chunk=chunk)
    n_splits = -(-used // chunk)
    pm = torch.empty((H_KV, n_splits, PAD_M), dtype=torch.float32, device="cuda")
    pl = torch.empty_like(pm)
    pa = torch.empty((H_KV, n_splits, PAD_M, D), dtype=torch.float32, device="cuda")
    out = torch.empty((1, HQ, 1, D), dtype=torch.float16, device="cuda")
    args = dict(used=used, chunk=chunk, scratch=(pm, pl, pa), out=out)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            int8_attn_decode(qc, *packed, **args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager_same_scratch = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        int8_attn_decode(qc, *packed, **args)
    for i in range(4):
        out.zero_()
        _ = int8_attn_decode(qc, *packed, used=used)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_same_scratch), f"replay {i}"
    assert_ulp_or_abs(npy(out)[0, :, 0], npy(want)[0, :, 0].astype(np.float64), 2.0, 1e-5, "scratch vs own")


def test_rejects_bad_inputs():
    """Error substrings of ``tests/test_kvattn.py:209-221``."""
    from nova_amd.kvattn import int8_attn_decode

    q, k, v = make(64)
    packed = _packed(k, v)
    qc = q.cuda()
    with pytest.raises(ValueError, match="解码一步"):
        int8_attn_decode(qc.expand(1, HQ, 2, D).contiguous(), *packed, used=64)
    with pytest.raises(ValueError, match="chunk"):
        int8_attn_decode(qc, *packed, used=64, chunk=100)
    with pytest.raises(ValueError, match="group"):
        int8_attn_decode(qc, *packed, used=64, group=100)
    with pytest.raises(ValueError, match="used"):
        int8_attn_decode(qc, *packed, used=65)
    with pytest.raises(ValueError, match="尺子"):
        int8_attn_decode(qc, *packed, used=64, group=32)


def test_device_scalars_match_python_ints():
    """``tests/test_kvattn_stream.py:217-230``: device-scalar and host-int launches agree bitwise."""
    from nova_amd.kvattn import GROUP_T, int8_attn_decode, pack_int8_kv

    used = 256
    k = randn((1, H_KV, used, D), 0)
    v = randn((1, H_KV, used, D), 1)
    q = randn((1, HQ, 1, D), 2).cuda()
    packed = pack_int8_kv(k.cuda(), v.cuda(), GROUP_T)
    a = int8_attn_decode(q, *packed, used=used, prefix_groups=used // GROUP_T)
    used_t = torch.tensor([used], dtype=torch.int64, device="cuda")
    pg_t = torch.tensor([used // GROUP_T], dtype=torch.int64, device="cuda")
    b = int8_attn_decode(q, *packed, used=None, used_t=used_t, prefix_groups_t=pg_t, n_splits=1)
    assert torch.equal(a, b)


def test_device_scalars_allow_partial_split():
    """Surplus splits of a capacity-sized launch see no tokens and must not inject 0/0."""
    from nova_amd.kvattn import GROUP_T, int8_attn_decode

    used = 320
    q, k, v = make(used)
    packed = _packed(k, v)
    n_splits = 4
    shape = (H_KV, n_splits, 16)
    pm = torch.zeros(shape, dtype=torch.float32, device="cuda")
    pl = torch.zeros_like(pm)
    pa = torch.zeros((*shape, D), dtype=torch.float32, device="cuda")
    out = torch.zeros(1, HQ, 1, D, dtype=torch.float16, device="cuda")
    lse = torch.zeros(1, HQ, dtype=torch.float32, device="cuda")
    qc = q.cuda()
    want = int8_attn_decode(qc, *packed, used=used, prefix_groups=used // GROUP_T)
    used_t = torch.tensor([used], dtype=torch.int64, device="cuda")
    pg_t = torch.tensor([used // GROUP_T], dtype=torch.int64, device="cuda")
    got = int8_attn_decode(qc, *packed, used=None, used_t=used_t, prefix_groups_t=pg_t, n_splits=n_splits,
                           scratch=(pm, pl, pa), out=out, lse_out=lse)
    assert torch.isfinite(got).all()
    assert_ulp_or_abs(npy(got)[0, :, 0], npy(want)[0, :, 0].astype(np.float64), 4.0, 1e-3, "partial split")


def test_prefix_groups_limits_the_scan():
    """``prefix_groups`` stops the scan at a whole ruler even when ``used`` is larger
    (``src/nova/kvattn.py:156-158``)."""
    from nova_amd.kvattn import int8_attn_decode

    q, k, v = make(500, seed=12)
    packed = _packed(k, v)
    got = int8_attn_decode(q.cuda(), *packed, used=500, prefix_groups=4)
    want, _ = _want(q, packed, 256)
    assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, "prefix_groups=4")


def test_long_context_layer_within_baseline_tolerance():
    """One layer of the 32768-token workload (K with 4 outlier channels x8 per head):
    max |out - oracle| <= 2e-3 and the reference's ULP criterion."""
    from nova_amd.kvattn import int8_attn_decode

    used = 32768
    k = bench_outliers(randn((1, H_KV, used, D), 100, 1.0), 101)
    v = randn((1, H_KV, used, D), 102, 1.0)
    q = (randn((1, HQ, 1, D), 103, 1.0).float() / D ** 0.5).half()
    packed = _packed(k, v)
    want, _ = _want(q, packed, used)
    got = npy(int8_attn_decode(q.cuda(), *packed, used=used))[0, :, 0]
    assert np.abs(got.astype(np.float64) - want.astype(np.float64)).max() <= 2e-3
    assert_ulp_or_abs(got, want, 2.0, 1e-5, "32k")


@pytest.mark.parametrize("gq", [1, 2, 8, 16])
def test_other_gqa_ratios(gq):
    from nova_amd.kvattn import int8_attn_decode

    hkv = 2
    used = 333
    q, k, v = make(used, seed=20 + gq, hq=hkv * gq, hkv=hkv)
    packed = _packed(k, v)
    want, _ = _want(q, packed, used)
    got = int8_attn_decode(q.cuda(), *packed, used=used)
    assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, f"gq={gq}")


def _steer(k: torch.Tensor, q: torch.Tensor, profile: str) -> torch.Tensor:
    """K with scores shaped along each KV head's first q head: ``jump`` adds 40 q/|q| to one
    token 300 before the end (its score passes every earlier one by ~40 in log2 units, far
    beyond the softmax's rescale headroom); ``rise`` adds a ramp 0 .. 20 q/|q| over the
    tokens (the reference maximum moves again and again)."""
    kf, qf = k.float(), q.float()[0, :, 0]
    n, gq = kf.shape[2], qf.shape[0] // kf.shape[1]
    for h in range(kf.shape[1]):
        dirv = qf[h * gq] / qf[h * gq].norm()
        if profile == "jump":
            kf[0, h, n - 300] += 40.0 * dirv
        else:
            kf[0, h] += torch.linspace(0.0, 20.0, n)[:, None] * dirv[None, :]
    return kf.half()


@pytest.mark.parametrize("profile", ["jump", "rise"])
def test_scores_that_move_the_softmax_reference(profile):
    """The online softmax moves its reference maximum only past a headroom; scores built to
    force a late large move, or many small ones, meet the ULP criterion against the oracle."""
    from nova_amd.kvattn import int8_attn_decode

    used = 4096
    q, k, v = make(used, seed=71)
    k = _steer(k, q, profile)
    packed = _packed(k, v)
    want, _ = _want(q, packed, used)
    got = int8_attn_decode(q.cuda(), *packed, used=used)
    assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, profile)
