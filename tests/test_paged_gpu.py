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
