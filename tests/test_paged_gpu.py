"""GPU parity of the paged batch decode (int8t64 pages, ragged sequences).

Each sequence of a paged batch must evolve exactly like a contiguous ``KVInt8Cache`` fed
the same tokens (codes, rulers and ring bit for bit), and its decode output must meet the
int8 criterion against that cache's output (<= 2 fp16 ULP or 1e-5: the same arithmetic,
split into different partial sums). The pages are handed out in a scrambled order so the
page-table indirection is exercised.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import D, H_KV, HQ, assert_ulp_or_abs, npy, randn

pytestmark = pytest.mark.gpu

LAYERS = 2


def _data(lens, steps, seed):
    ks = [randn((1, H_KV, n + steps, D), seed + 10 * b) for b, n in enumerate(lens)]
    vs = [randn((1, H_KV, n + steps, D), seed + 10 * b + 5) for b, n in enumerate(lens)]
    qs = [randn((len(lens), HQ, 1, D), seed + 1000 + i) for i in range(steps)]
    return [k.cuda() for k in ks], [v.cuda() for v in vs], [q.cuda() for q in qs]


def _paged(lens, steps, ks, vs, seed):
    from nova_amd.paged import PagedKVInt8Cache

    per_seq = max(-(-(n + steps + 1) // 64) for n in lens)
    cache = PagedKVInt8Cache(LAYERS, H_KV, D, HQ, max_seqs=len(lens), num_pages=per_seq * len(lens) + 3,
                             max_pages_per_seq=per_seq)
    rng = np.random.default_rng(seed)
    cache._free = [int(x) for x in rng.permutation(cache.num_pages)]
    for b, n in enumerate(lens):
        cache.reserve(b, n + steps + 1)
        for layer in range(LAYERS):
            cache.prefill(b, layer, ks[b][:, :, :n], vs[b][:, :, :n])
    cache.plan()
    return cache


def _contiguous(n, steps, k, v):
    from nova_amd.kvattn import KVInt8Cache

    c = KVInt8Cache(num_slots=LAYERS, num_kv_heads=H_KV, head_dim=D, max_len=n + steps + 64, num_q_heads=HQ)
    c.begin_prefill(n)
    c.set_prefill_pos(0)
    for layer in range(LAYERS):
        c.update(k[:, :, :n], v[:, :, :n], layer)
    c.finish_prefill(n)
    return c


def _check_state(paged, conts, lens, step):
    for b, c in enumerate(conts):
        upto = (lens[b] + step) // 64 + 1  # groups written so far, the current one included
        for layer in range(LAYERS):
            pg = paged.pages[layer]
            for g in range(upto):
                page = int(paged.page_table[b, g])
                for i, (q, st, mn) in enumerate(((c.kq, c.kst, c.kmn), (c.vq, c.vst, c.vmn))):
                    want = q[layer][0, :, 64 * g:64 * g + 64].reshape(H_KV, -1)
                    assert torch.equal(pg[page, :, i * 8192:(i + 1) * 8192], want), (b, layer, g, i)
                    base = 16384 + i * 512
                    assert torch.equal(pg[page, :, base:base + 256].view(torch.float16), st[layer][0, :, g]), (b, g, i)
                    assert torch.equal(pg[page, :, base + 256:base + 512].view(torch.float16), mn[layer][0, :, g])
            assert torch.equal(paged.rings[layer][b, :, 0], c.tail_k[layer][0]), (b, layer)
            assert torch.equal(paged.rings[layer][b, :, 1], c.tail_v[layer][0]), (b, layer)


def _set_parts(cache, parts):
    """A caller's own work plan, as the C entry points accept it: ``parts[b]`` prefix parts
    for sequence b (here fewer than ``plan()`` gives, down to one part per sequence)."""
    wg_map, seq_parts = [], []
    for b, p in enumerate(parts):
        seq_parts += [len(wg_map), p]
        wg_map += [(b << 16) | i for i in range(p)]
    cache.wg_map = torch.tensor(wg_map, dtype=torch.int32, device="cuda")
    cache.seq_parts = torch.tensor(seq_parts, dtype=torch.int32, device="cuda")
    cache.total_parts = len(wg_map)


@pytest.mark.parametrize("lens,parts,steps", [([70, 200, 1000, 64], None, 70), ([1, 63, 129], None, 70),
                                              ([70, 200, 1000, 64], [1, 2, 3, 1], 70),
                                              ([9000, 13000, 4600], None, 3)])  # the benchmark's scale
def test_paged_batch_matches_contiguous_caches(lens, parts, steps):
    print(f"case lens={lens} parts={parts}", flush=True)
    ks, vs, qs = _data(lens, steps, seed=40)
    paged = _paged(lens, steps, ks, vs, seed=41)
    if parts is not None:
        _set_parts(paged, parts)
    conts = [_contiguous(n, steps, ks[b], vs[b]) for b, n in enumerate(lens)]
    _check_state(paged, conts, lens, -1)
    for i in range(steps):
        for layer in range(LAYERS):
            kn = torch.cat([ks[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
            vn = torch.cat([vs[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
            out = paged.decode_step(kn, vn, qs[i], layer).clone()
            for b, (n, c) in enumerate(zip(lens, conts)):
                c.pos.fill_(n + i)
                want = c.update_attend(ks[b][:, :, n + i:n + i + 1], vs[b][:, :, n + i:n + i + 1],
                                       qs[i][b:b + 1], layer)
                assert_ulp_or_abs(npy(out[b, :, 0]), npy(want[0, :, 0]).astype(np.float64), 2.0, 1e-5,
                                  f"b={b} step={i} layer={layer}")
        paged.advance()
        if i in (0, 1, steps - 1) or (i % 17 == 0):
            _check_state(paged, conts, lens, i)


def test_paged_graph_replay_equals_eager():
    lens, steps = [90, 300, 65], 20
    ks, vs, qs = _data(lens, steps, seed=50)
    e = _paged(lens, steps, ks, vs, seed=51)
    g = _paged(lens, steps, ks, vs, seed=51)
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
        kn = torch.cat([ks[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
        vn = torch.cat([vs[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
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
        assert torch.equal(e.rings[layer], g.rings[layer])


def _bench_lengths():
    """The batched ragged decode configuration's 8 sequence lengths (seed 3, uniform in [1024, 16384])."""
    return [int(x) for x in torch.randint(1024, 16385, (8,), generator=torch.Generator().manual_seed(3))]


def test_paged_bench_batch_against_oracle():
    """The batched ragged configuration itself: the benchmark's 8 seeded lengths (4.6k-13.7k
    tokens), 2 layers x 3 decode steps, every sequence's output against the oracle's single
    softmax over its own int8 prefix and fp16 ring (the streaming criterion: 4 ULP or 1e-3)."""
    from oracle import stream as ostream

    lens, steps = _bench_lengths(), 3
    print(f"case lens={lens}", flush=True)
    ks, vs, qs = _data(lens, steps, seed=60)
    paged = _paged(lens, steps, ks, vs, seed=61)
    outs = torch.empty(steps, LAYERS, len(lens), HQ, 1, D, dtype=torch.float16, device="cuda")
    for i in range(steps):
        kn = torch.cat([ks[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
        vn = torch.cat([vs[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
        for layer in range(LAYERS):
            outs[i, layer].copy_(paged.decode_step(kn, vn, qs[i], layer))
        paged.advance()
    torch.cuda.synchronize()
    got = npy(outs)
    q_all = np.stack([npy(q) for q in qs])  # [steps, B, HQ, 1, D]
    for b, n in enumerate(lens):
        want = ostream.decode_trajectory(npy(ks[b])[0], npy(vs[b])[0], q_all[:, b, :, 0], n)
        for layer in range(LAYERS):  # the layers hold the same tokens in separate page pools
            for i in range(steps):
                assert_ulp_or_abs(got[i, layer, b, :, 0], want[i], 4.0, 1e-3, f"b={b} n={n} layer={layer} step={i}")


def test_bucket_padding_is_never_read():
    """The reference pads a sequence's capacity to its bucket (src/nova/decode.py:39-48) and
    masks the padding to -inf (decode.py:200-205). Here the padding is never read: with every
    sequence's pages reserved up to bucket_for(its length), the padded pages and the ring slots
    holding positions already in the int8 prefix filled with garbage, decoding gives outputs
    identical bit for bit to a cache without padding."""
    from nova_amd.decode import bucket_for

    lens, steps = [1000, 2100, 70, 4100], 70
    ks, vs, qs = _data(lens, steps, seed=70)
    plain = _paged(lens, steps, ks, vs, seed=71)
    from nova_amd.paged import PagedKVInt8Cache

    per_seq = max(-(-bucket_for(n + steps + 1) // 64) for n in lens)
    padded = PagedKVInt8Cache(LAYERS, H_KV, D, HQ, max_seqs=len(lens), num_pages=per_seq * len(lens),
                              max_pages_per_seq=per_seq)
    g = torch.Generator(device="cuda").manual_seed(72)
    for b, n in enumerate(lens):
        padded.reserve(b, bucket_for(n + steps + 1))
        for layer in range(LAYERS):
            pool = padded.pages[layer]
            pool.copy_(torch.randint(0, 256, pool.shape, generator=g, device="cuda", dtype=torch.uint8))
    for b, n in enumerate(lens):
        for layer in range(LAYERS):
            padded.prefill(b, layer, ks[b][:, :, :n], vs[b][:, :, :n])
            # stale ring slots (positions already in the int8 prefix) get garbage too
            for i in range(64):
                pos = (n - 1) - ((n - 1 - i) % 64)
                if pos < n // 64 * 64:
                    padded.rings[layer][b, :, :, i] = torch.randn(H_KV, 2, D, generator=g, device="cuda").half() * 50
    padded.plan(lens)
    _set_parts(padded, [int(plain.seq_parts[2 * b + 1]) for b in range(len(lens))])
    for i in range(steps):
        kn = torch.cat([ks[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
        vn = torch.cat([vs[b][:, :, n + i:n + i + 1] for b, n in enumerate(lens)], 0)
        for layer in range(LAYERS):
            a = plain.decode_step(kn, vn, qs[i], layer).clone()
            p = padded.decode_step(kn, vn, qs[i], layer)
            assert torch.equal(a, p), (i, layer)
            assert torch.equal(plain.lse[:len(lens)], padded.lse[:len(lens)]), (i, layer)
        plain.advance()
        padded.advance()


def test_released_sequence_appends_and_attends_nothing():
    """A released sequence's table row is -1: a plan that still names it neither writes into the
    pages (which may now belong to another sequence) nor reads them; its output is 0."""
    lens, steps = [300, 500], 2
    ks, vs, qs = _data(lens, steps, seed=80)
    cache = _paged(lens, steps, ks, vs, seed=81)
    before = [p.clone() for p in cache.pages]
    cache.release(1)
    kn = torch.cat([ks[b][:, :, n:n + 1] for b, n in enumerate(lens)], 0)
    vn = torch.cat([vs[b][:, :, n:n + 1] for b, n in enumerate(lens)], 0)
    cache.pos[1] = lens[1]  # a stale position, as a plan captured before the release would hold
    out = cache.decode_step(kn, vn, qs[0], 0).clone()
    torch.cuda.synchronize()
    assert int(out[1].abs().sum()) == 0 and bool(torch.isinf(cache.lse[1]).all())
    assert torch.isfinite(out[0]).all() and float(out[0].abs().sum()) > 0
    changed = (cache.pages[0] != before[0]).any(dim=2).any(dim=1).nonzero().flatten().tolist()
    assert set(changed) <= set(cache._owned[0]), "only sequence 0's pages may change"
