"""GPU parity of the paged batch in the per-token symmetric format (``PagedKVInt8TokCache``).

Every sequence of a paged batch must hold exactly the codes and scales a contiguous
``KVInt8TokCache`` holds for the same tokens, bit for bit, and its decode output must meet
the int8 criterion against that cache's output (<= 2 fp16 ULP or 1e-5: the same arithmetic,
split into different partial sums) and the oracle's (dequantize, then one softmax: 4 ULP or
1e-3). Pages are handed out in a scrambled order so the page-table indirection is exercised.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import D, H_KV, HQ, assert_ulp_or_abs, npy
from tests.test_paged_gpu import LAYERS, _bench_lengths, _data, _set_parts

pytestmark = pytest.mark.gpu

PAGE = 16640
CODE = 64 * D


def _paged(lens, steps, ks, vs, seed, pad_to=None):
    from nova_amd.paged import PagedKVInt8TokCache

    need = [-(-((pad_to(n + steps + 1) if pad_to else n + steps + 1)) // 64) for n in lens]
    per_seq = max(need)
    cache = PagedKVInt8TokCache(LAYERS, H_KV, D, HQ, max_seqs=len(lens), num_pages=sum(need) + 3,
                                max_pages_per_seq=per_seq)
    rng = np.random.default_rng(seed)
    cache._free = [int(x) for x in rng.permutation(cache.num_pages)]
    for b, n in enumerate(lens):
        cache.reserve(b, 64 * need[b])
    return cache


def _fill(cache, lens, ks, vs):
    for b, n in enumerate(lens):
        for layer in range(LAYERS):
            cache.prefill(b, layer, ks[b][:, :, :n], vs[b][:, :, :n])
    cache.plan()


def _contiguous(n, steps, k, v):
    from nova_amd.kvtok import KVInt8TokCache

    c = KVInt8TokCache(num_slots=LAYERS, num_kv_heads=H_KV, head_dim=D, max_len=n + steps + 64, num_q_heads=HQ)
    c.begin_prefill(n)
    c.set_prefill_pos(0)
    for layer in range(LAYERS):
        c.update(k[:, :, :n], v[:, :, :n], layer)
    c.finish_prefill(n)
    return c


def _gather(cache, layer, b, upto):
    """Sequence b's tokens [0, upto) of one layer, read back from its pages: K codes, V codes
    ``[H_kv, upto, 128]`` int8 and K, V scales ``[H_kv, upto]`` fp16."""
    pg = cache.pages[layer]
    groups = -(-upto // 64)
    rows = torch.stack([pg[int(cache.page_table[b, g])] for g in range(groups)], 1)  # [H_kv, G, PAGE]
    kq = rows[:, :, :CODE].reshape(H_KV, groups * 64, D)[:, :upto].view(torch.int8)
    vq = rows[:, :, CODE:2 * CODE].reshape(H_KV, groups * 64, D)[:, :upto].view(torch.int8)
    sc = rows[:, :, 2 * CODE:].contiguous().view(torch.float16).reshape(H_KV, groups, 2, 64)
    ksc = sc[:, :, 0].reshape(H_KV, groups * 64)[:, :upto]
    vsc = sc[:, :, 1].reshape(H_KV, groups * 64)[:, :upto]
    return kq, vq, ksc, vsc


def _check_state(paged, conts, lens, written):
    for b, c in enumerate(conts):
        upto = lens[b] + written
        for layer in range(LAYERS):
            kq, vq, ksc, vsc = _gather(paged, layer, b, upto)
            assert torch.equal(kq, c.kq[layer][0, :, :upto]), (b, layer, "kq")
            assert torch.equal(vq, c.vq[layer][0, :, :upto]), (b, layer, "vq")
            assert torch.equal(ksc, c.ksc[layer][0, :, :upto]), (b, layer, "ksc")
            assert torch.equal(vsc, c.vsc[layer][0, :, :upto]), (b, layer, "vsc")


def _step_inputs(ks, vs, lens, i):
    kn = torch.cat([ks[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
    vn = torch.cat([vs[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
    return kn, vn


@pytest.mark.parametrize("lens,parts,steps", [([70, 200, 1000, 64], None, 70), ([1, 63, 129], None, 70),
                                              ([70, 200, 1000, 64], [1, 2, 3, 1], 70),
                                              ([9000, 13000, 4600], None, 3)])
def test_tok_pages_match_contiguous_caches(lens, parts, steps):
    print(f"case tok pages lens={lens} parts={parts}", flush=True)
    ks, vs, qs = _data(lens, steps, seed=140)
    paged = _paged(lens, steps, ks, vs, seed=141)
    _fill(paged, lens, ks, vs)
    if parts is not None:
        _set_parts(paged, parts)
    conts = [_contiguous(n, steps, ks[b], vs[b]) for b, n in enumerate(lens)]
    _check_state(paged, conts, lens, 0)
    for i in range(steps):
        kn, vn = _step_inputs(ks, vs, lens, i)
        for layer in range(LAYERS):
            out = paged.decode_step(kn, vn, qs[i], layer).clone()
            for b, (n, c) in enumerate(zip(lens, conts)):
                c.pos.fill_(n + i)
                want = c.update_attend(ks[b][:, :, n + i:n + i + 1], vs[b][:, :, n + i:n + i + 1],
                                       qs[i][b:b + 1], layer)
                assert_ulp_or_abs(npy(out[b, :, 0]), npy(want[0, :, 0]).astype(np.float64), 2.0, 1e-5,
                                  f"b={b} step={i} layer={layer}")
        paged.advance()
        if i in (0, 1, steps - 1) or i % 17 == 0:
            _check_state(paged, conts, lens, i + 1)


def test_tok_paged_bench_batch_against_oracle():
    """The batched ragged configuration's 8 seeded lengths (4.6k-13.7k tokens), 2 layers x 3
    decode steps, every output against the oracle: per-token symmetric quantization of every
    token up to and including the step's, dequantization, one softmax (4 ULP or 1e-3)."""
    from oracle import attn as oattn
    from oracle import kvquant as okq

    lens, steps = _bench_lengths(), 3
    print(f"case tok pages lens={lens}", flush=True)
    ks, vs, qs = _data(lens, steps, seed=160)
    paged = _paged(lens, steps, ks, vs, seed=161)
    _fill(paged, lens, ks, vs)
    outs = torch.empty(steps, LAYERS, len(lens), HQ, 1, D, dtype=torch.float16, device="cuda")
    for i in range(steps):
        kn, vn = _step_inputs(ks, vs, lens, i)
        for layer in range(LAYERS):
            outs[i, layer].copy_(paged.decode_step(kn, vn, qs[i], layer))
        paged.advance()
    torch.cuda.synchronize()
    got = npy(outs)
    for b, n in enumerate(lens):
        kq, ksc = okq.quantize_tok(npy(ks[b])[0])
        vq, vsc = okq.quantize_tok(npy(vs[b])[0])
        for i in range(steps):
            want, _ = oattn.tok_attn_decode(npy(qs[i])[b, :, 0], kq, ksc, vq, vsc, n + i + 1)
            for layer in range(LAYERS):  # the layers hold the same tokens in separate page pools
                assert_ulp_or_abs(got[i, layer, b, :, 0], want.astype(np.float64), 4.0, 1e-3,
                                  f"b={b} n={n} layer={layer} step={i}")


def test_tok_paged_quantize_in_chunks_at_any_offset():
    """A prompt stored in two chunks split inside a page (tokens [0, 100) then [100, 777)) gives
    the pages of one call, which hold the contiguous quantizer's codes and scales."""
    from nova_amd import _lib
    from nova_amd.kvtok import quantize_tok

    n = 777
    ks, vs, _ = _data([n], 0, seed=170)
    one = _paged([n], 0, ks, vs, seed=171)
    two = _paged([n], 0, ks, vs, seed=171)
    one.prefill(0, 0, ks[0], vs[0])
    row = two.page_table[0]
    for which, x in enumerate((ks[0], vs[0])):
        for c0, c1 in ((0, 100), (100, n)):
            xc = x[0, :, c0:c1].contiguous()
            _lib.call("nkv_paged_quantize_tok", xc.data_ptr(), 0, xc.stride(0), H_KV, c1 - c0, which,
                      two.pages[0].data_ptr(), row.data_ptr(), c0, two.num_pages, _lib.stream_ptr(row.device))
    torch.cuda.synchronize()
    assert torch.equal(one.pages[0], two.pages[0])
    kq, vq, ksc, vsc = _gather(one, 0, 0, n)
    wk, wks = quantize_tok(ks[0])
    wv, wvs = quantize_tok(vs[0])
    assert torch.equal(kq, wk[0]) and torch.equal(ksc, wks[0].view(torch.float16).reshape(H_KV, n))
    assert torch.equal(vq, wv[0]) and torch.equal(vsc, wvs[0].view(torch.float16).reshape(H_KV, n))


def test_tok_paged_graph_replay_equals_eager():
    lens, steps = [90, 300, 65], 20
    ks, vs, qs = _data(lens, steps, seed=150)
    e = _paged(lens, steps, ks, vs, seed=151)
    g = _paged(lens, steps, ks, vs, seed=151)
    _fill(e, lens, ks, vs)
    _fill(g, lens, ks, vs)
    B = len(lens)
    k_in = torch.empty(B, H_KV, 1, D, dtype=torch.float16, device="cuda")
    v_in = torch.empty_like(k_in)
    q_in = torch.empty(B, HQ, 1, D, dtype=torch.float16, device="cuda")
    outs = [torch.empty(B, HQ, 1, D, dtype=torch.float16, device="cuda") for _ in range(LAYERS)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for layer in range(LAYERS):
                outs[layer].copy_(g.decode_step(k_in, v_in, q_in, layer))
            g.pos[:B].add_(1)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(steps):
        kn, vn = _step_inputs(ks, vs, lens, i)
        k_in.copy_(kn)
        v_in.copy_(vn)
        q_in.copy_(qs[i])
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(LAYERS):
            want = e.decode_step(kn, vn, qs[i], layer)
            assert torch.equal(outs[layer], want), (i, layer)
        e.advance()
        torch.cuda.synchronize()
    for layer in range(LAYERS):
        assert torch.equal(e.pages[layer], g.pages[layer])


def test_tok_bucket_padding_is_never_read():
    """Pages reserved up to each sequence's bucket (src/nova/decode.py:39-48) and filled with
    garbage beyond the prompt: decoding gives outputs identical bit for bit to pages without
    padding (the positions the reference masks to -inf, decode.py:200-205, are not read)."""
    from nova_amd.decode import bucket_for

    lens, steps = [1000, 2100, 70, 4100], 70
    ks, vs, qs = _data(lens, steps, seed=180)
    plain = _paged(lens, steps, ks, vs, seed=181)
    _fill(plain, lens, ks, vs)
    padded = _paged(lens, steps, ks, vs, seed=182, pad_to=bucket_for)
    g = torch.Generator(device="cuda").manual_seed(183)
    for layer in range(LAYERS):
        pool = padded.pages[layer]
        pool.copy_(torch.randint(0, 256, pool.shape, generator=g, device="cuda", dtype=torch.uint8))
    _fill(padded, lens, ks, vs)
    _set_parts(padded, [int(plain.seq_parts[2 * b + 1]) for b in range(len(lens))])
    for i in range(steps):
        kn, vn = _step_inputs(ks, vs, lens, i)
        for layer in range(LAYERS):
            a = plain.decode_step(kn, vn, qs[i], layer).clone()
            p = padded.decode_step(kn, vn, qs[i], layer)
            assert torch.equal(a, p), (i, layer)
            assert torch.equal(plain.lse[:len(lens)], padded.lse[:len(lens)]), (i, layer)
        plain.advance()
        padded.advance()


def test_tok_released_sequence_appends_and_attends_nothing():
    """A released sequence's table row is -1: a plan that still names it neither writes into the
    pages nor reads them; its output is 0 and its lse -inf."""
    lens, steps = [300, 500], 2
    ks, vs, qs = _data(lens, steps, seed=190)
    cache = _paged(lens, steps, ks, vs, seed=191)
    _fill(cache, lens, ks, vs)
    before = [p.clone() for p in cache.pages]
    cache.release(1)
    kn, vn = _step_inputs(ks, vs, lens, 0)
    cache.pos[1] = lens[1]  # a stale position, as a plan captured before the release would hold
    out = cache.decode_step(kn, vn, qs[0], 0).clone()
    torch.cuda.synchronize()
    assert int(out[1].abs().sum()) == 0 and bool(torch.isinf(cache.lse[1]).all())
    assert torch.isfinite(out[0]).all() and float(out[0].abs().sum()) > 0
    changed = (cache.pages[0] != before[0]).any(dim=2).any(dim=1).nonzero().flatten().tolist()
    assert set(changed) <= set(cache._owned[0]), "only sequence 0's pages may change"
