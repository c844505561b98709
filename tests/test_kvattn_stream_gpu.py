"""GPU parity of the streaming int8 cache — restates the reference's
``tests/test_kvattn_stream.py`` and adds bit-exact state checks against the oracle
and against the reference's own trajectory (``tests/golden/stream.npz``).

Output criterion (``tests/test_kvattn_stream.py:39-57``): <= 4 fp16 ULP or <= 1e-3
absolute against "int8 prefix dequantized + fp16 tail, one softmax".
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from oracle import kvquant as okq
from oracle import stream as ostream
from tests.helpers import D, H_KV, HQ, assert_ulp_or_abs, make, npy, randn

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
MAX_ULP, ABS_TOL = 4.0, 1e-3


def _cache(slots: int = 1, max_len: int = 512, hq: int = HQ, hkv: int = H_KV):
    from nova_amd.kvattn import KVInt8Cache

    return KVInt8Cache(num_slots=slots, num_kv_heads=hkv, head_dim=D, max_len=max_len, num_q_heads=hq)


def _prefill_then_last(cache, k, v, q, layer: int = 0, chunk: int = 0, fused: bool = False):
    """First L-1 tokens prefilled, the L-th appended as one decode step
    (``tests/test_kvattn_stream.py:91-107``)."""
    k, v, q = k.cuda(), v.cuda(), q.cuda()
    L = k.shape[2]
    n0 = L - 1
    cache.begin_prefill(n0)
    if chunk:
        for c0 in range(0, n0, chunk):
            nc = min(chunk, n0 - c0)
            cache.set_prefill_pos(c0)
            cache.update(k[:, :, c0:c0 + nc], v[:, :, c0:c0 + nc], layer)
    else:
        cache.set_prefill_pos(0)
        cache.update(k[:, :, :n0], v[:, :, :n0], layer)
    cache.finish_prefill(n0)
    cache.pos.fill_(L - 1)
    if fused:
        return cache.update_attend(k[:, :, L - 1:], v[:, :, L - 1:], q, layer)
    cache.update(k[:, :, L - 1:], v[:, :, L - 1:], layer)
    return cache.attend(q, layer)


def _reference(k, v, q, used: int, prefix: int) -> np.ndarray:
    """Prefix ``[0, prefix)`` through the int8t64 round trip, the rest fp16, one softmax
    (``tests/test_kvattn_stream.py:68-83``)."""
    kn, vn = npy(k)[0], npy(v)[0]
    if prefix:
        kq, kmn, kst = okq.quantize_int8_token(kn[:, :prefix], 64)
        vq, vmn, vst = okq.quantize_int8_token(vn[:, :prefix], 64)
        kk = np.concatenate([okq.dequantize_int8_token(kq, kmn, kst, 64), kn[:, prefix:used]], axis=1)
        vv = np.concatenate([okq.dequantize_int8_token(vq, vmn, vst, 64), vn[:, prefix:used]], axis=1)
    else:
        kk, vv = kn[:, :used], vn[:, :used]
    out, _ = oattn.attend_fp16_kv(npy(q)[0, :, 0], kk, vv)
    return out


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("used", [40, 64, 100, 128, 192, 320])
def test_matches_dequant_then_attention(used, fused):
    print(f"case used={used} fused={fused}", flush=True)
    q, k, v = make(used)
    cache = _cache()
    got = _prefill_then_last(cache, k, v, q, fused=fused)
    want = _reference(k, v, q, used, used // 64 * 64)
    assert_ulp_or_abs(npy(got)[0, :, 0], want, MAX_ULP, ABS_TOL, f"used={used}")
    assert int(cache._qlen.item()) == used // 64 * 64


def test_prefix_grows_with_pos():
    q, k, v = make(128)
    cache = _cache()
    k, v = k.cuda(), v.cuda()
    cache.begin_prefill(63)
    cache.set_prefill_pos(0)
    cache.update(k[:, :, :63], v[:, :, :63], 0)
    cache.finish_prefill(63)
    assert int(cache._qlen.item()) == 0
    for p in range(63, 128):
        cache.pos.fill_(p)
        cache.update(k[:, :, p:p + 1], v[:, :, p:p + 1], 0)
        assert int(cache._qlen.item()) == (p + 1) // 64 * 64, p
        assert int(cache._written.item()) == p + 1
        assert int(cache._pg.item()) == (p + 1) // 64


def test_ring_mask_excludes_prefix():
    q, k, v = make(200)
    cache = _cache()
    k, v = k.cuda(), v.cuda()
    cache.begin_prefill(199)
    cache.set_prefill_pos(0)
    cache.update(k[:, :, :199], v[:, :, :199], 0)
    cache.finish_prefill(199)
    cache.pos.fill_(199)
    cache.update(k[:, :, 199:], v[:, :, 199:], 0)
    mask = cache.ring_mask().view(-1).cpu()
    qlen, written = int(cache._qlen.item()), int(cache._written.item())
    idx = torch.arange(64)
    abs_pos = (written - 1) - torch.remainder((written - 1) - idx, 64)
    for i in range(64):
        if bool(mask[i]):
            assert qlen <= int(abs_pos[i]) < written
    assert bool(mask.any())
    assert int(mask.sum()) == written - qlen


@pytest.mark.parametrize("chunk", [64, 96, 128])
def test_prefill_multi_block_equals_single(chunk):
    used = 300
    q, k, v = make(used)
    one = _prefill_then_last(_cache(), k, v, q)
    chunked = _prefill_then_last(_cache(), k, v, q, chunk=chunk)
    assert torch.equal(one, chunked)


def test_finish_prefill_matches_quantizer():
    from nova_amd.kvquant import quantize_int8

    used = 192
    _, k, v = make(used)
    k, v = k.cuda(), v.cuda()
    cache = _cache()
    cache.begin_prefill(used)
    cache.set_prefill_pos(0)
    cache.update(k, v, 0)
    cache.finish_prefill(used)
    kq, kmn, kst = quantize_int8(k, 64, "token")
    vq, vmn, vst = quantize_int8(v, 64, "token")
    assert torch.equal(cache.kq[0][:, :, :used], kq)
    assert torch.equal(cache.vq[0][:, :, :used], vq)
    n = used // 64
    assert torch.equal(cache.kmn[0][:, :, :n], kmn) and torch.equal(cache.kst[0][:, :, :n], kst)
    assert torch.equal(cache.vmn[0][:, :, :n], vmn) and torch.equal(cache.vst[0][:, :, :n], vst)
    assert cache.staging is None


def test_slots_are_independent():
    used = 200
    q, k0, v0 = make(used)
    k1, v1 = randn(k0.shape, 99, 1.0), randn(v0.shape, 98, 1.0)
    cache = _cache(slots=2)
    k0c, v0c, k1c, v1c, qc = k0.cuda(), v0.cuda(), k1.cuda(), v1.cuda(), q.cuda()
    cache.begin_prefill(used - 1)
    cache.set_prefill_pos(0)
    cache.update(k0c[:, :, :used - 1], v0c[:, :, :used - 1], 0)
    cache.update(k1c[:, :, :used - 1], v1c[:, :, :used - 1], 1)
    cache.finish_prefill(used - 1)
    cache.pos.fill_(used - 1)
    cache.update(k0c[:, :, used - 1:], v0c[:, :, used - 1:], 0)
    cache.update(k1c[:, :, used - 1:], v1c[:, :, used - 1:], 1)
    got0 = cache.attend(qc, 0).clone()
    got1 = cache.attend(qc, 1).clone()
    p = used // 64 * 64
    assert_ulp_or_abs(npy(got0)[0, :, 0], _reference(k0, v0, q, used, p), MAX_ULP, ABS_TOL, "slot 0")
    assert_ulp_or_abs(npy(got1)[0, :, 0], _reference(k1, v1, q, used, p), MAX_ULP, ABS_TOL, "slot 1")
    assert not torch.equal(got0, got1)


def test_short_context_is_all_fp16():
    used = 33
    q, k, v = make(used)
    cache = _cache()
    got = _prefill_then_last(cache, k, v, q)
    assert int(cache._qlen.item()) == 0
    assert torch.isfinite(got).all()
    assert_ulp_or_abs(npy(got)[0, :, 0], _reference(k, v, q, used, 0), MAX_ULP, ABS_TOL, "prefix=0")


def test_tail_attend_matches_oracle():
    from nova_amd.kvattn import tail_attend

    q = randn((1, HQ, 1, D), 1).cuda()
    k = randn((1, H_KV, 64, D), 2).cuda()
    v = randn((1, H_KV, 64, D), 3).cuda()
    for bits in (0, (1 << 64) - 1, 0x00ff00000000ff01, 1 << 63):
        mask = torch.tensor([(bits >> i) & 1 for i in range(64)], dtype=torch.bool).view(1, 1, 1, 64).cuda()
        out, lse = tail_attend(q, k, v, mask)
        wo, wl = oattn.tail_attend(npy(q)[0, :, 0], npy(k)[0], npy(v)[0], npy(mask).reshape(-1))
        assert_ulp_or_abs(npy(out)[0, :, 0], wo, 2.0, 1e-5, f"mask={bits:x}")
        np.testing.assert_allclose(npy(lse)[0], wl, rtol=1e-5, atol=1e-5)


def _state_equal(cache, ref: ostream.StreamCache, layer: int = 0, tag: str = ""):
    assert np.array_equal(npy(cache.kq[layer])[0], ref.kq[layer]), tag
    assert np.array_equal(npy(cache.vq[layer])[0], ref.vq[layer]), tag
    for nm in ("kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
        assert np.array_equal(npy(getattr(cache, nm)[layer])[0].view(np.uint16),
                              getattr(ref, nm)[layer].view(np.uint16)), f"{tag} {nm}"
    assert [int(cache._written.item()), int(cache._qlen.item()), int(cache._pg.item())] == \
        [ref.written, ref.qlen, ref.pg], tag


@pytest.mark.parametrize("fused", [False, True])
def test_reference_trajectory_bit_exact(fused):
    """Replay the reference's own chunked prefill + 70 appends (``tests/golden/stream.npz``):
    codes, rulers, ring and scalars equal the reference's at every recorded point."""
    z = np.load(GOLD / "stream.npz")
    k, v, q = (torch.from_numpy(z[n]).cuda() for n in ("k", "v", "q"))
    n0, max_len = int(z["n0"]), int(z["max_len"])
    cache = _cache(max_len=max_len, hq=q.shape[1], hkv=k.shape[1])
    cache.begin_prefill(n0)
    for c0 in range(0, n0, 96):
        nc = min(96, n0 - c0)
        cache.set_prefill_pos(c0)
        cache.update(k[:, :, c0:c0 + nc], v[:, :, c0:c0 + nc], 0)
    cache.finish_prefill(n0)

    def check(tag):
        assert np.array_equal(npy(cache.kq[0]), z[f"{tag}_kq"]), tag
        assert np.array_equal(npy(cache.vq[0]), z[f"{tag}_vq"]), tag
        for nm in ("kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
            assert np.array_equal(npy(getattr(cache, nm)[0]).view(np.uint16), z[f"{tag}_{nm}"].view(np.uint16)), nm

    check("prefill")
    for i in range(z["step_scalars"].shape[0]):
        p = n0 + i
        cache.pos.fill_(p)
        if fused:
            cache.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0)
        else:
            cache.update(k[:, :, p:p + 1], v[:, :, p:p + 1], 0)
        assert [int(cache._written.item()), int(cache._qlen.item()), int(cache._pg.item())] == \
            list(z["step_scalars"][i]), p
        assert np.array_equal(npy(cache.ring_mask()).reshape(-1), z["step_masks"][i]), p
        if f"step{p}_kq" in z:
            check(f"step{p}")


def test_fused_equals_two_calls():
    """``update_attend`` leaves the same state as ``update`` and returns ``attend``'s
    output within the streaming criterion, across group boundaries."""
    used0 = 120
    _, k, v = make(used0 + 80, seed=31)
    q = randn((1, HQ, 1, D), 32).cuda()
    k, v = k.cuda(), v.cuda()
    a, b = _cache(max_len=256), _cache(max_len=256)
    for c in (a, b):
        c.begin_prefill(used0)
        c.set_prefill_pos(0)
        c.update(k[:, :, :used0], v[:, :, :used0], 0)
        c.finish_prefill(used0)
    for p in range(used0, used0 + 80):
        a.pos.fill_(p)
        b.pos.fill_(p)
        a.update(k[:, :, p:p + 1], v[:, :, p:p + 1], 0)
        oa = a.attend(q, 0).clone()
        ob = b.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0).clone()
        for nm in ("kq", "vq", "kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
            assert torch.equal(getattr(a, nm)[0], getattr(b, nm)[0]), (p, nm)
        for nm in ("_written", "_qlen", "_pg"):
            assert torch.equal(getattr(a, nm), getattr(b, nm)), (p, nm)
        assert_ulp_or_abs(npy(ob)[0, :, 0], npy(oa)[0, :, 0].astype(np.float64), MAX_ULP, ABS_TOL, f"p={p}")


def test_partials_then_combine_equals_fused_step():
    """The decode step's two launches called one by one (``nkv_decode_step_partials_t64``
    then ``nkv_decode_step_combine_t64``) give the fused call's state and output bit for
    bit, across a group boundary and with more parts than groups."""
    from nova_amd import _lib

    used0 = 190
    _, k, v = make(used0 + 70, seed=37)
    q = randn((1, HQ, 1, D), 38).cuda()
    k, v = k.cuda(), v.cuda()
    a, b = _cache(max_len=320), _cache(max_len=320)
    for c in (a, b):
        c.begin_prefill(used0)
        c.set_prefill_pos(0)
        c.update(k[:, :, :used0], v[:, :, :used0], 0)
        c.finish_prefill(used0)
    for p in range(used0, used0 + 70):
        a.pos.fill_(p)
        b.pos.fill_(p)
        oa = a.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0).clone()
        args = b.step_args(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0)
        _lib.call("nkv_decode_step_partials_t64", *args)
        _lib.call("nkv_decode_step_combine_t64", *args)
        ob = b.merged.clone()
        for nm in ("kq", "vq", "kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
            assert torch.equal(getattr(a, nm)[0], getattr(b, nm)[0]), (p, nm)
        for nm in ("_written", "_qlen", "_pg"):
            assert torch.equal(getattr(a, nm), getattr(b, nm)), (p, nm)
        assert torch.equal(oa, ob), p
        assert torch.equal(a.lse, b.lse), p


def test_fused_step_at_32k_context():
    """The decode step at the benchmark's context (32 parts per KV head over 512 groups),
    across the 512th group boundary: the fused step equals its two launches called one by
    one bit for bit (state and output), the two-call ``update`` + ``attend`` within the
    streaming criterion, and the dequantize-then-attend oracle likewise."""
    from nova_amd import _lib

    used0, steps = 32766, 4
    _, k, v = make(used0 + steps, seed=61)
    q = randn((1, HQ, 1, D), 62).cuda()
    k, v = k.cuda(), v.cuda()
    caches = [_cache(max_len=used0 + 128) for _ in range(3)]
    for c in caches:
        c.begin_prefill(used0)
        c.set_prefill_pos(0)
        c.update(k[:, :, :used0], v[:, :, :used0], 0)
        c.finish_prefill(used0)
    fused, split, two = caches
    for p in range(used0, used0 + steps):
        print(f"case 32k step pos={p}", flush=True)
        for c in caches:
            c.pos.fill_(p)
        kn, vn = k[:, :, p:p + 1], v[:, :, p:p + 1]
        of = fused.update_attend(kn, vn, q, 0).clone()
        args = split.step_args(kn, vn, q, 0)
        _lib.call("nkv_decode_step_partials_t64", *args)
        _lib.call("nkv_decode_step_combine_t64", *args)
        two.update(kn, vn, 0)
        ot = two.attend(q, 0).clone()
        for nm in ("kq", "vq", "kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
            assert torch.equal(getattr(fused, nm)[0], getattr(split, nm)[0]), (p, nm)
            assert torch.equal(getattr(fused, nm)[0], getattr(two, nm)[0]), (p, nm)
        assert torch.equal(of, split.merged), p
        assert_ulp_or_abs(npy(of)[0, :, 0], npy(ot)[0, :, 0].astype(np.float64), MAX_ULP, ABS_TOL, f"two-call p={p}")
        qlen = int(fused._qlen.item())
        assert qlen == (p + 1) // 64 * 64
        want = _reference(k, v, q, p + 1, qlen)
        assert_ulp_or_abs(npy(of)[0, :, 0], want, MAX_ULP, ABS_TOL, f"oracle p={p}")


def test_fused_tail_leaves_the_workspace_zero_and_layers_interleave():
    """The fused step publishes each partial word by word into the zero-filled workspace and
    its merger sets every word it consumed back to zero, as does the split's tail kernel:
    after every call the whole workspace reads zero. Two caches of different lengths and
    several layers interleave on one stream, each call checked against the two-launch split
    (partials, then the tail kernel), bit for bit."""
    from nova_amd import _lib
    from nova_amd.kvattn import KVInt8Cache

    layers, used0 = 3, (130, 700)
    caches, ref = [], []
    data = []
    for i, n in enumerate(used0):
        _, k, v = make(n + 40, seed=60 + i)
        data.append((k.cuda(), v.cuda()))
        pair = []
        for _ in range(2):
            c = KVInt8Cache(num_slots=layers, num_kv_heads=H_KV, head_dim=D, max_len=n + 128, num_q_heads=HQ)
            c.begin_prefill(n)
            c.set_prefill_pos(0)
            for layer in range(layers):
                c.update(data[i][0][:, :, :n], data[i][1][:, :, :n], layer)
            c.finish_prefill(n)
            pair.append(c)
        caches.append(pair[0])
        ref.append(pair[1])
    for step in range(40):
        q = randn((1, HQ, 1, D), 900 + step).cuda()
        for layer in range(layers):
            for i, n in enumerate(used0):
                k, v = data[i]
                p = n + step
                a, b = caches[i], ref[i]
                a.pos.fill_(p)
                b.pos.fill_(p)
                oa = a.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, layer).clone()
                args = b.step_args(k[:, :, p:p + 1], v[:, :, p:p + 1], q, layer)
                _lib.call("nkv_decode_step_partials_t64", *args)
                _lib.call("nkv_decode_step_combine_t64", *args)
                assert torch.equal(oa, b.merged), (step, layer, i)
                assert torch.equal(a.lse, b.lse), (step, layer, i)
        for c in caches + ref:
            assert int(torch.count_nonzero(c._ws)) == 0, step


def test_streaming_decode_4096_steps_against_oracle():
    """The streaming workload, one layer: prefill 512, then 4096 fused append + attend steps
    (q ~ N(0,1)/sqrt(128)). Every step's output is checked against the oracle's single-softmax
    value (the batched trajectory oracle, pinned on the CPU against the state machine), and the
    cache state equals the oracle's bit for bit at the end."""
    n0, steps = 512, 4096
    g = torch.Generator().manual_seed(1)
    k = torch.randn(1, H_KV, n0 + steps, D, generator=g).half()
    v = torch.randn(1, H_KV, n0 + steps, D, generator=g).half()
    qs = (torch.randn(steps, 1, HQ, 1, D, generator=g) / D ** 0.5).half()
    kc, vc, qc = k.cuda(), v.cuda(), qs.cuda()
    cache = _cache(max_len=n0 + steps)
    cache.begin_prefill(n0)
    cache.set_prefill_pos(0)
    cache.update(kc[:, :, :n0], vc[:, :, :n0], 0)
    cache.finish_prefill(n0)
    outs = torch.empty(steps, 1, HQ, 1, D, dtype=torch.float16, device="cuda")
    for i in range(steps):
        cache.pos.fill_(n0 + i)
        p = n0 + i
        cache.update_attend(kc[:, :, p:p + 1], vc[:, :, p:p + 1], qc[i], 0, out=outs[i])
    torch.cuda.synchronize()
    kn, vn = npy(k)[0], npy(v)[0]
    want = ostream.decode_trajectory(kn, vn, npy(qs)[:, 0, :, 0], n0)
    got = npy(outs)[:, 0, :, 0]
    for i in range(steps):
        assert_ulp_or_abs(got[i], want[i], MAX_ULP, ABS_TOL, f"step {i}")
    ref = ostream.StreamCache(1, H_KV, D, n0 + steps, HQ)
    ref.begin_prefill(n0)
    ref.set_prefill_pos(0)
    ref.update(kn[:, :n0], vn[:, :n0], 0)
    ref.finish_prefill(n0)
    for i in range(steps):
        ref.pos = n0 + i
        ref.update(kn[:, n0 + i:n0 + i + 1], vn[:, n0 + i:n0 + i + 1], 0)
    _state_equal(cache, ref, 0, "after 4096 steps")


def test_graph_capture_of_decode_steps():
    """Capture one fused step (+ ``pos += 1``), replay it over 70 positions with fresh K/V
    copied in between; outputs and state equal an eager twin cache bit for bit."""
    used0 = 150
    _, k, v = make(used0 + 70, seed=41)
    q = randn((1, HQ, 1, D), 42).cuda()
    k, v = k.cuda(), v.cuda()
    g_cache, e_cache = _cache(max_len=256), _cache(max_len=256)
    for c in (g_cache, e_cache):
        c.begin_prefill(used0)
        c.set_prefill_pos(0)
        c.update(k[:, :, :used0], v[:, :, :used0], 0)
        c.finish_prefill(used0)
    k_in = k[:, :, used0:used0 + 1].clone()
    v_in = v[:, :, used0:used0 + 1].clone()
    # warm up on a copy of the state, then restore (as GraphDecoder.capture does)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_cache.update_attend(k_in, v_in, q, 0)
        g_cache.pos.add_(1)
    for i in range(70):
        p = used0 + i
        k_in.copy_(k[:, :, p:p + 1])
        v_in.copy_(v[:, :, p:p + 1])
        graph.replay()
        e_cache.pos.fill_(p)
        want = e_cache.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0)
        torch.cuda.synchronize()
        assert torch.equal(g_cache.merged, want), p
        assert int(g_cache.pos.item()) == p + 1
    for nm in ("kq", "vq", "kmn", "kst", "tail_k", "tail_v"):
        assert torch.equal(getattr(g_cache, nm)[0], getattr(e_cache, nm)[0]), nm


def test_cuda_graph_capture_attend():
    """``tests/test_kvattn_stream.py:259-277``: attend captured, replays equal eager."""
    used = 200
    q, k, v = make(used)
    cache = _cache(max_len=256)
    eager = _prefill_then_last(cache, k, v, q).clone()
    kc, vc, qc = k.cuda(), v.cuda(), q.cuda()
    cache.pos.fill_(used - 1)
    cache.update(kc[:, :, used - 1:], vc[:, :, used - 1:], 0)
    cache.refresh_scalars()
    g = torch.cuda.CUDAGraph()
    with torch.inference_mode():
        with torch.cuda.graph(g):
            cache.attend(qc, 0)
    for _ in range(3):
        cache.merged.zero_()
        with torch.inference_mode():
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(cache.merged, eager)


def test_nbytes_ratio():
    """int8 resident bytes vs fp16 at 2048 slots (``tests/test_graph_decode_int8.py:73-85``)."""
    c = _cache(slots=2, max_len=2048)
    ratio = c.nbytes() / c.fp16_nbytes()
    assert 0.4 < ratio < 0.6
    ref = ostream.StreamCache(2, H_KV, D, 2048, HQ)
    assert c.nbytes() == ref.nbytes()
