"""GPU parity of the per-token symmetric int8 format ("tok"): quantizer, decode attention
and streaming cache against the oracle (``oracle.kvquant.quantize_tok`` /
``oracle.attn.tok_attn_decode``).

Codes and scales must be bit-exact. Attention uses the int8 criterion of the reference's
decode-attention tests (``tests/test_kvattn.py:80-93``): every element within 2 fp16 ULP
or 1e-5 absolute of "dequantize, then softmax attention" (fp64 oracle).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from oracle import kvquant as okq
from tests.helpers import D, H_KV, HQ, assert_ulp_or_abs, bench_outliers, make, npy, randn
from tests.test_oracle import TOK_SPECIAL_CODES, TOK_SPECIAL_SCALES, _tok_special_rows

pytestmark = pytest.mark.gpu


def _quant_cases():
    g = torch.Generator().manual_seed(11)
    base = torch.randn(2, 3, 37, D, generator=g)
    yield "f16", (base * 2.0).to(torch.float16)
    yield "bf16", (base * 0.3).to(torch.bfloat16)
    yield "f32", base * 5.0
    x = (base * 1.5).to(torch.float16)
    x[0, 0, 3] = 0.0                      # an all-zero row: scale floor, codes 0
    x[0, 1, 4] = 2.5                      # a constant row: every code 127
    x[1, 2, 5, 7] = 6.0e4                 # one huge value per row
    x[1, 0, 6] = (torch.arange(D) - 64).to(torch.float16) * 1e-3   # tiny magnitudes
    yield "special", x
    yield "outliers", bench_outliers(randn((1, H_KV, 96, D), 12), seed=13)
    yield "rounding", torch.from_numpy(_tok_special_rows()).reshape(1, 1, 2, D)


@pytest.mark.parametrize("case", [c for c, _ in _quant_cases()])
def test_quantize_tok_bit_exact(case):
    from nova_amd.kvtok import dequantize_tok, quantize_tok

    x = dict(_quant_cases())[case]
    q, s = quantize_tok(x.cuda())
    wq, ws = okq.quantize_tok(x.float().numpy() if x.dtype == torch.bfloat16 else x.numpy())
    np.testing.assert_array_equal(npy(q), wq)
    np.testing.assert_array_equal(npy(s).view(np.uint16), ws.view(np.uint16))
    deq = dequantize_tok(q, s)
    np.testing.assert_array_equal(npy(deq).view(np.uint16), okq.dequantize_tok(wq, ws).view(np.uint16))
    if case == "rounding":  # the literal codes and scales (round half to even, fp32 scale)
        for r in range(2):
            n = len(TOK_SPECIAL_CODES[r])
            assert npy(q)[0, 0, r, :n].tolist() == TOK_SPECIAL_CODES[r]
            assert not npy(q)[0, 0, r, n:].any()
            assert int(npy(s)[0, 0, r:r + 1].view(np.uint16)[0]) == TOK_SPECIAL_SCALES[r]


def test_quantize_tok_strided_slabs():
    """A slab view with a row stride quantizes like its contiguous copy."""
    from nova_amd.kvtok import quantize_tok

    big = randn((1, 4, 80, D), 14).cuda()
    view = big[:, :, 10:70]
    q1, s1 = quantize_tok(view)
    q2, s2 = quantize_tok(view.contiguous())
    assert torch.equal(q1, q2) and torch.equal(s1, s2)


def _tok_cache_tensors(k, v, cap):
    from nova_amd.kvtok import quantize_tok

    kq, ks = quantize_tok(k.cuda())
    vq, vs = quantize_tok(v.cuda())
    used = k.shape[2]
    pad = cap - used

    def grow(t, fill=0):
        shape = list(t.shape)
        shape[2] = pad
        return torch.cat([t, torch.full(shape, fill, dtype=t.dtype, device=t.device)], 2).contiguous()

    return grow(kq), grow(ks), grow(vq), grow(vs)


@pytest.mark.parametrize("used", [1, 31, 64, 65, 500, 2048, 4097])
def test_tok_attention_against_oracle(used):
    from nova_amd.kvtok import int8_tok_attn_decode

    print(f"case used={used}", flush=True)
    q, k, v = make(used, seed=20)
    cap = -(-used // 64) * 64 + 64
    kq, ks, vq, vs = _tok_cache_tensors(k, v, cap)
    lse = torch.empty(1, HQ, device="cuda", dtype=torch.float32)
    got = int8_tok_attn_decode(q.cuda(), kq, ks, vq, vs, used=used, lse_out=lse)
    want, want_lse = oattn.tok_attn_decode(npy(q)[0, :, 0], npy(kq)[0], npy(ks)[0], npy(vq)[0], npy(vs)[0], used)
    st = assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, f"used={used}")
    assert st["exact"] > 0.95, st
    np.testing.assert_allclose(npy(lse)[0], want_lse, rtol=0, atol=2e-5)


def test_tok_single_layer_2048_with_outliers():
    """Quantize + one decode step, 32 q / 8 kv heads, context 2048, 4 seeded K channels per
    head x8, fp16 N(0,1) inputs."""
    from nova_amd.kvtok import int8_tok_attn_decode

    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, H_KV, 2048, D, generator=g).to(torch.float16)
    v = torch.randn(1, H_KV, 2048, D, generator=g).to(torch.float16)
    q = (torch.randn(1, HQ, 1, D, generator=g) / D ** 0.5).to(torch.float16)
    k = bench_outliers(k, seed=1)
    kq, ks, vq, vs = _tok_cache_tensors(k, v, 2048)
    got = int8_tok_attn_decode(q.cuda(), kq, ks, vq, vs, used=2048)
    wq, ws = okq.quantize_tok(k.numpy())
    np.testing.assert_array_equal(npy(kq)[0], wq[0])
    want, _ = oattn.tok_attn_decode(npy(q)[0, :, 0], wq[0], ws[0], *(a[0] for a in okq.quantize_tok(v.numpy())), 2048)
    assert_ulp_or_abs(npy(got)[0, :, 0], want, 2.0, 1e-5, "cfg1")
    # the reference's own tolerance for the whole int8 path against exact fp16 attention
    exact, _ = oattn.attend_fp16_kv(npy(q)[0, :, 0], npy(k)[0], npy(v)[0])
    assert np.abs(npy(got)[0, :, 0].astype(np.float64) - exact).max() <= 2e-3


def test_tok_used_zero_and_device_length():
    from nova_amd.kvtok import int8_tok_attn_decode

    q, k, v = make(300, seed=21)
    kq, ks, vq, vs = _tok_cache_tensors(k, v, 320)
    lse = torch.empty(1, HQ, device="cuda")
    out = int8_tok_attn_decode(q.cuda(), kq, ks, vq, vs, used=0, lse_out=lse)
    assert torch.count_nonzero(out) == 0 and torch.isneginf(lse).all()
    a = int8_tok_attn_decode(q.cuda(), kq, ks, vq, vs, used=257).clone()
    b = int8_tok_attn_decode(q.cuda(), kq, ks, vq, vs, used_t=torch.tensor([257], device="cuda"))
    assert torch.equal(a, b)


def _stream(cache, k, v, q, n0, steps, fused):
    cache.begin_prefill(n0)
    cache.set_prefill_pos(0)
    cache.update(k[:, :, :n0], v[:, :, :n0], 0)
    cache.finish_prefill(n0)
    outs = []
    for p in range(n0, n0 + steps):
        cache.pos.fill_(p)
        if fused:
            outs.append(cache.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0).clone())
        else:
            cache.update(k[:, :, p:p + 1], v[:, :, p:p + 1], 0)
            outs.append(cache.attend(q, 0).clone())
    return outs


def test_tok_streaming_cache_against_oracle():
    """Prefill 150 tokens, then 80 decode steps: the cache holds exactly the oracle's codes
    and scales of every token, and each step's output meets the criterion; the fused step
    and the two-call sequence agree bit for bit in state and to 2 ULP in output."""
    from nova_amd.kvtok import KVInt8TokCache

    n0, steps = 150, 80
    _, k, v = make(n0 + steps, seed=22)
    q = randn((1, HQ, 1, D), 23).cuda()
    k, v = k.cuda(), v.cuda()
    a = KVInt8TokCache(1, H_KV, D, 256, HQ)
    b = KVInt8TokCache(1, H_KV, D, 256, HQ)
    oa = _stream(a, k, v, q, n0, steps, fused=False)
    ob = _stream(b, k, v, q, n0, steps, fused=True)
    for nm in ("kq", "vq", "ksc", "vsc"):
        assert torch.equal(getattr(a, nm)[0], getattr(b, nm)[0]), nm
    assert int(b._written.item()) == n0 + steps
    wkq, wks = okq.quantize_tok(npy(k))
    wvq, wvs = okq.quantize_tok(npy(v))
    n = n0 + steps
    np.testing.assert_array_equal(npy(b.kq[0])[:, :, :n], wkq)
    np.testing.assert_array_equal(npy(b.ksc[0])[:, :, :n].view(np.uint16), wks.view(np.uint16))
    np.testing.assert_array_equal(npy(b.vq[0])[:, :, :n], wvq)
    for i, p in enumerate(range(n0, n0 + steps)):
        want, _ = oattn.tok_attn_decode(npy(q)[0, :, 0], wkq[0], wks[0], wvq[0], wvs[0], p + 1)
        assert_ulp_or_abs(npy(ob[i])[0, :, 0], want, 2.0, 1e-5, f"fused p={p}")
        assert_ulp_or_abs(npy(oa[i])[0, :, 0], want, 2.0, 1e-5, f"two-call p={p}")


def test_tok_graph_replay_equals_eager():
    from nova_amd.kvtok import KVInt8TokCache

    n0, steps = 100, 12
    _, k, v = make(n0 + steps, seed=24)
    q = randn((1, HQ, 1, D), 25).cuda()
    k, v = k.cuda(), v.cuda()
    e = KVInt8TokCache(1, H_KV, D, 192, HQ)
    g = KVInt8TokCache(1, H_KV, D, 192, HQ)
    for c in (e, g):
        c.begin_prefill(n0)
        c.set_prefill_pos(0)
        c.update(k[:, :, :n0], v[:, :, :n0], 0)
        c.finish_prefill(n0)
    k_in = torch.empty(1, H_KV, 1, D, dtype=torch.float16, device="cuda")
    v_in = torch.empty_like(k_in)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            g.update_attend(k_in, v_in, q, 0)
            g.pos.add_(1)
    torch.cuda.current_stream().wait_stream(s)
    g.pos.fill_(n0)
    for p in range(n0, n0 + steps):
        k_in.copy_(k[:, :, p:p + 1])
        v_in.copy_(v[:, :, p:p + 1])
        graph.replay()
        torch.cuda.synchronize()
        e.pos.fill_(p)
        want = e.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0)
        torch.cuda.synchronize()
        assert torch.equal(g.merged, want), p
    for nm in ("kq", "vq", "ksc", "vsc"):
        assert torch.equal(getattr(e, nm)[0], getattr(g, nm)[0]), nm


def test_tok_partials_then_combine_equals_fused_step():
    from nova_amd import _lib
    from nova_amd.kvtok import KVInt8TokCache

    n0 = 130
    _, k, v = make(n0 + 5, seed=26)
    q = randn((1, HQ, 1, D), 27).cuda()
    k, v = k.cuda(), v.cuda()
    a, b = KVInt8TokCache(1, H_KV, D, 192, HQ), KVInt8TokCache(1, H_KV, D, 192, HQ)
    for c in (a, b):
        c.begin_prefill(n0)
        c.set_prefill_pos(0)
        c.update(k[:, :, :n0], v[:, :, :n0], 0)
        c.finish_prefill(n0)
    for p in range(n0, n0 + 5):
        a.pos.fill_(p)
        b.pos.fill_(p)
        oa = a.update_attend(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0).clone()
        args = b.step_args(k[:, :, p:p + 1], v[:, :, p:p + 1], q, 0)
        _lib.call("nkv_decode_step_partials_tok", *args)
        _lib.call("nkv_decode_step_combine_tok", *args)
        assert torch.equal(oa, b.merged), p
        assert torch.equal(a.lse, b.lse), p
        for nm in ("kq", "vq", "ksc", "vsc"):
            assert torch.equal(getattr(a, nm)[0], getattr(b, nm)[0]), (p, nm)
