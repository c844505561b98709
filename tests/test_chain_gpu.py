"""GPU parity of the chained decode step (``nkv_decode_layers_t64`` / ``_tok``): every layer of
one token in one launch, each layer's inputs views of the previous layer's output, under both
dependency modes (``dep="all"``: every layer waits for every head of the layer before;
``dep="head"``: forwarded inputs wait only for their own head).

Each layer is checked against the oracle applied to the inputs that layer actually received
(so float differences do not compound along the chain): the cache state bit for bit against
``oracle.stream.StreamCache`` (int8t64) or ``oracle.kvquant.quantize_tok`` (per-token
symmetric), every output within the streaming criterion of ``tests/test_kvattn_stream.py:39-57``
(<= 4 fp16 ULP or <= 1e-3; per-token symmetric: the int8 criterion, 2 ULP or 1e-5). Against
the per-layer launches (``nkv_decode_step_t64``) the state is bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from oracle import kvquant as okq
from oracle import stream as ostream
from tests.helpers import D, H_KV, HQ, assert_ulp_or_abs, bench_outliers, npy, randn

pytestmark = pytest.mark.gpu

GQ = HQ // H_KV
MAX_ULP, ABS_TOL = 4.0, 1e-3


def _chain_views(outs: torch.Tensor, layers: int):
    """Layer l reads layer l - 1's output (layer 0: the last layer's, from the step before):
    q = the whole output, k = its q heads 0, 4, .., v = its q heads 1, 5, .."""
    qs = [outs[(l - 1) % layers] for l in range(layers)]
    ks = [q[:, 0::GQ] for q in qs]
    vs = [q[:, 1::GQ] for q in qs]
    return ks, vs, qs, [outs[l] for l in range(layers)]


def _prefill_t64(cache, layers: int, n0: int, seed: int, oracle=None):
    cache.begin_prefill(n0)
    cache.set_prefill_pos(0)
    if oracle is not None:
        oracle.begin_prefill(n0)
        oracle.set_prefill_pos(0)
    for l in range(layers):
        k = bench_outliers(randn((1, H_KV, n0, D), seed + 10 * l), seed + 10 * l + 1)
        v = randn((1, H_KV, n0, D), seed + 10 * l + 2)
        cache.update(k.cuda(), v.cuda(), l)
        if oracle is not None:
            oracle.update(npy(k)[0], npy(v)[0], l)
    cache.finish_prefill(n0)
    if oracle is not None:
        oracle.finish_prefill(n0)


def _assert_state(cache, oracle, layers: int):
    for l in range(layers):
        for nm in ("kq", "vq"):
            np.testing.assert_array_equal(npy(getattr(cache, nm)[l])[0], getattr(oracle, nm)[l], err_msg=f"{nm}[{l}]")
        for nm in ("kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
            np.testing.assert_array_equal(npy(getattr(cache, nm)[l])[0].view(np.uint16),
                                          getattr(oracle, nm)[l].view(np.uint16), err_msg=f"{nm}[{l}]")
    assert int(cache._written.item()) == oracle.written
    assert int(cache._qlen.item()) == oracle.qlen
    assert int(cache._pg.item()) == oracle.pg


@pytest.mark.parametrize("dep", ["all", "head"])
@pytest.mark.parametrize("n_parts,L,n0,steps,cap", [(0, 3, 250, 72, 512), (3, 3, 250, 72, 512), (3, 2, 1750, 48, 2048)])
def test_chain_t64_against_oracle(n_parts, L, n0, steps, cap, dep):
    """Chained layers from a prefill of n0 tokens, then steps across group boundaries (250: the
    boundaries at 256 and 320, one or two halves per wave; 1750 over 3 parts: 9 and then 10
    groups per part, so that waves take two or three halves): every layer's output against the
    oracle on its own inputs, state bit for bit."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    print(f"case chain t64 n_parts={n_parts} L={L} n0={n0} steps={steps} dep={dep}", flush=True)
    cache = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    ref = ostream.StreamCache(L, H_KV, D, cap, HQ)
    _prefill_t64(cache, L, n0, seed=40, oracle=ref)
    outs = randn((L, 1, HQ, 1, D), 41, scale=0.5).cuda()
    chain = ChainedStep(cache, *_chain_views(outs, L), n_parts=n_parts, dep=dep)
    for s in range(steps):
        prev = npy(outs)  # layer 0's input is outs[L - 1] before the step
        chain()
        got = npy(outs)
        for l in range(L):
            q = (prev if l == 0 else got)[(l - 1) % L][0, :, 0]
            ref.update(q[0::GQ, None], q[1::GQ, None], l)
            want = ref.attend_exact(q, l)
            assert_ulp_or_abs(got[l][0, :, 0], want, MAX_ULP, ABS_TOL, f"step {s} layer {l}")
        cache.pos.add_(1)
        ref.pos += 1
    _assert_state(cache, ref, L)
    assert chain.idle_state() == {"partials_zero": True, "counters_zero": True, "error": 0, "launches": steps}
    chain.check()


@pytest.mark.parametrize("dep", ["all", "head"])
def test_chain_cross_head_inputs(dep):
    """Head h's new K token taken from KV head h + 1's rows of the previous layer's output (the
    outputs padded by one KV head's rows, which head 7 reads as zeros), so the mergers' inputs
    are not forwarded and wait for every head: with dep="all" at every layer, layer 0 included
    (it reads the previous step's layer 2 output, overwritten later in the launch); with
    dep="head" from layer 1 on (layer 0's k is head-local). Every output against the oracle on
    its own inputs, state bit for bit."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    print(f"case chain cross-head dep={dep}", flush=True)
    L, n0, steps, cap = 3, 600, 40, 1024
    cache = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    ref = ostream.StreamCache(L, H_KV, D, cap, HQ)
    _prefill_t64(cache, L, n0, seed=90, oracle=ref)
    pad = torch.zeros(L, 1, HQ + GQ, 1, D, dtype=torch.float16, device="cuda")
    pad[:, :, :HQ] = randn((L, 1, HQ, 1, D), 91, scale=0.5).cuda()
    outs = [pad[l, :, :HQ] for l in range(L)]
    qs = [outs[(l - 1) % L] for l in range(L)]
    cross = lambda l: dep == "all" or l > 0  # noqa: E731
    ks = [pad[(l - 1) % L, :, (GQ if cross(l) else 0)::GQ][:, :H_KV] for l in range(L)]
    vs = [pad[(l - 1) % L, :, 1::GQ][:, :H_KV] for l in range(L)]
    chain = ChainedStep(cache, ks, vs, qs, outs, dep=dep)
    for s in range(steps):
        prev = npy(pad)
        chain()
        got = npy(pad)
        for l in range(L):
            src = (prev if l == 0 else got)[(l - 1) % L][0, :, 0]
            q = src[:HQ]
            k = src[GQ::GQ] if cross(l) else src[0:HQ:GQ]
            ref.update(k[:, None], src[1:HQ:GQ, None], l)
            want = ref.attend_exact(q, l)
            assert_ulp_or_abs(got[l][0, :HQ, 0], want, MAX_ULP, ABS_TOL, f"step {s} layer {l}")
        cache.pos.add_(1)
        ref.pos += 1
    _assert_state(cache, ref, L)
    chain.check()


@pytest.mark.parametrize("dep", ["all", "head"])
def test_chain_bench_configuration(dep):
    """The configuration the long-context benchmark times: 36 layers at 32k context (a prefill of
    32765 tokens, so the 3 steps cross the 512th group boundary), the default grid, every layer's
    q / k / v views of the previous layer's output. Every layer of every step against the per-layer
    fused launches (``update_attend``) of a second cache fed the same inputs: state bit-identical,
    outputs within the streaming criterion; one deep layer against the oracle; no wait gave up."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    print(f"case chain bench configuration dep={dep}", flush=True)
    L, n0, cap = 36, 32765, 32768 + 128
    dev = torch.device("cuda")
    caches = [KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ) for _ in range(2)]
    for c in caches:
        c.begin_prefill(n0)
        c.set_prefill_pos(0)
    gen = torch.Generator(device=dev).manual_seed(80)
    cpu_gen = torch.Generator().manual_seed(81)
    for l in range(L):
        k = torch.randn(1, H_KV, n0, D, generator=gen, device=dev)
        for h in range(H_KV):
            k[0, h, :, torch.randperm(D, generator=cpu_gen)[:4].to(dev)] *= 8.0
        k, v = k.half(), torch.randn(1, H_KV, n0, D, generator=gen, device=dev).half()
        for c in caches:
            c.update(k, v, l)
        del k, v
    for c in caches:
        c.finish_prefill(n0)
    a, b = caches
    outs = (torch.randn(L, 1, HQ, 1, D, generator=gen, device=dev) / D ** 0.5).half()
    ob = torch.zeros_like(outs)
    chain = ChainedStep(a, *_chain_views(outs, L), dep=dep)
    assert chain.n_parts >= 16
    for step in range(3):
        last = outs[L - 1].clone()  # layer 0's input: the previous step's last output
        chain()
        for l in range(L):
            src = last if l == 0 else outs[l - 1]
            b.update_attend(src[:, 0::GQ], src[:, 1::GQ], src, l, out=ob[l])
        got, want = npy(outs), npy(ob)
        for l in range(L):
            assert_ulp_or_abs(got[l][0, :, 0], want[l][0, :, 0].astype(np.float64), MAX_ULP, ABS_TOL,
                              f"step {step} layer {l}")
        a.pos.add_(1)
        b.pos.add_(1)
        for nm in ("_codes", "_rulers", "_ring", "_scalars"):
            assert torch.equal(getattr(a, nm), getattr(b, nm)), f"{nm} after step {step}"
    # the last step's layer 27 against the oracle: its state dequantized, one softmax over it
    deep = 27
    ref = ostream.StreamCache(1, H_KV, D, cap, HQ)
    ref.kq[0], ref.vq[0] = npy(a.kq[deep])[0], npy(a.vq[deep])[0]
    for nm in ("kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
        getattr(ref, nm)[0] = npy(getattr(a, nm)[deep])[0]
    ref.pos = int(a.pos.item()) - 1
    ref._sync_scalars()
    want = ref.attend_exact(npy(outs[deep - 1])[0, :, 0], 0)
    assert_ulp_or_abs(npy(outs[deep])[0, :, 0], want, MAX_ULP, ABS_TOL, "layer 27 vs oracle")
    assert not chain.gave_up()
    chain.check()


def test_chain_equals_per_layer_launches_at_32k():
    """2 layers at 32768 tokens with the default grid (one workgroup per CU), 3 steps across
    the 512th group boundary, independent inputs: cache state bit-identical to the per-layer
    fused launches, outputs within the streaming criterion of them and of the oracle."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    print("case chain 32k", flush=True)
    L, n0, cap = 2, 32765, 32768 + 128
    a = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    b = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    _prefill_t64(a, L, n0, seed=50)
    _prefill_t64(b, L, n0, seed=50)
    dev = torch.device("cuda")
    qs = [randn((1, HQ, 1, D), 51 + l, 0.5).to(dev) for l in range(L)]
    ks = [randn((1, H_KV, 1, D), 53 + l).to(dev) for l in range(L)]
    vs = [randn((1, H_KV, 1, D), 55 + l).to(dev) for l in range(L)]
    oa = [torch.zeros(1, HQ, 1, D, dtype=torch.float16, device=dev) for _ in range(L)]
    ob = [torch.zeros_like(o) for o in oa]
    chain = ChainedStep(a, ks, vs, qs, oa)
    assert chain.n_parts >= 16
    for step in range(3):
        chain()
        for l in range(L):
            b.update_attend(ks[l], vs[l], qs[l], l, out=ob[l])
        for l in range(L):
            assert_ulp_or_abs(npy(oa[l])[0, :, 0], npy(ob[l])[0, :, 0].astype(np.float64), MAX_ULP, ABS_TOL,
                              f"step {step} layer {l}")
        a.pos.add_(1)
        b.pos.add_(1)
        for nm in ("_codes", "_rulers", "_ring", "_scalars"):
            assert torch.equal(getattr(a, nm), getattr(b, nm)), f"{nm} after step {step}"
    # the last step against the oracle: layer 1's state, dequantized, one softmax
    ref = ostream.StreamCache(1, H_KV, D, cap, HQ)
    ref.kq[0], ref.vq[0] = npy(a.kq[1])[0], npy(a.vq[1])[0]
    for nm in ("kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
        getattr(ref, nm)[0] = npy(getattr(a, nm)[1])[0]
    ref.pos = int(a.pos.item()) - 1
    ref._sync_scalars()
    want = ref.attend_exact(npy(qs[1])[0, :, 0], 0)
    assert_ulp_or_abs(npy(oa[1])[0, :, 0], want, MAX_ULP, ABS_TOL, "32k vs oracle")
    assert not chain.gave_up()


def test_chain_graph_replay_equals_eager():
    """The chained step captured with ``pos += 1`` in a graph, replayed, equals eager calls bit
    for bit (outputs and state), with eager work between the replays."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    print("case chain graph", flush=True)
    L, n0, cap = 4, 1000, 1280
    caches, outs, chains = [], [], []
    for _ in range(2):
        c = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
        _prefill_t64(c, L, n0, seed=60)
        o = randn((L, 1, HQ, 1, D), 61, scale=0.5).cuda()
        caches.append(c)
        outs.append(o)
        chains.append(ChainedStep(c, *_chain_views(o, L)))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g):
            chains[1]()
            caches[1].pos.add_(1)
    torch.cuda.current_stream().wait_stream(side)
    for step in range(30):
        chains[0]()
        caches[0].pos.add_(1)
        g.replay()
        _ = torch.randn(1000, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), f"outputs differ at step {step}"
    for nm in ("_codes", "_rulers", "_ring", "_scalars"):
        assert torch.equal(getattr(caches[0], nm), getattr(caches[1], nm)), nm


@pytest.mark.parametrize("dep", ["all", "head"])
@pytest.mark.parametrize("n_parts,n0,steps,cap", [(0, 190, 70, 320), (3, 1750, 48, 2048), (1, 1200, 40, 1280)])
def test_chain_tok_against_oracle(n_parts, n0, steps, cap, dep):
    """Per-token symmetric caches, 2 chained layers, a prefill of n0 tokens and then steps that
    end at every offset within a group (190: one half per wave; 1750 over 3 parts: two or three
    halves per wave; 1200 in one part: four or five): codes and scales of every token bit for
    bit against the quantizer oracle, every output against the oracle."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvtok import KVInt8TokCache

    print(f"case chain tok n_parts={n_parts} n0={n0} steps={steps} dep={dep}", flush=True)
    L = 2
    cache = KVInt8TokCache(L, H_KV, D, cap, HQ)
    cache.begin_prefill(n0)
    cache.set_prefill_pos(0)
    ks_all, vs_all = [], []
    for l in range(L):
        k = bench_outliers(randn((1, H_KV, n0, D), 70 + l), 72 + l)
        v = randn((1, H_KV, n0, D), 74 + l)
        cache.update(k.cuda(), v.cuda(), l)
        ks_all.append([npy(k)[0]])
        vs_all.append([npy(v)[0]])
    cache.finish_prefill(n0)
    outs = randn((L, 1, HQ, 1, D), 76, scale=0.5).cuda()
    chain = ChainedStep(cache, *_chain_views(outs, L), n_parts=n_parts, dep=dep)
    for s in range(steps):
        prev = npy(outs)
        chain()
        got = npy(outs)
        p = n0 + s
        for l in range(L):
            q = (prev if l == 0 else got)[(l - 1) % L][0, :, 0]
            ks_all[l].append(q[0::GQ, None])
            vs_all[l].append(q[1::GQ, None])
            kq, ksc = okq.quantize_tok(np.concatenate(ks_all[l], axis=1))
            vq, vsc = okq.quantize_tok(np.concatenate(vs_all[l], axis=1))
            want, _ = oattn.tok_attn_decode(q, kq, ksc, vq, vsc, p + 1)
            assert_ulp_or_abs(got[l][0, :, 0], want, 2.0, 1e-5, f"step {s} layer {l}")
        cache.pos.add_(1)
    n = n0 + steps
    for l in range(L):
        kq, ksc = okq.quantize_tok(np.concatenate(ks_all[l], axis=1))
        vq, vsc = okq.quantize_tok(np.concatenate(vs_all[l], axis=1))
        np.testing.assert_array_equal(npy(cache.kq[l])[0, :, :n], kq)
        np.testing.assert_array_equal(npy(cache.vq[l])[0, :, :n], vq)
        np.testing.assert_array_equal(npy(cache.ksc[l])[0, :, :n].view(np.uint16), ksc.view(np.uint16))
        np.testing.assert_array_equal(npy(cache.vsc[l])[0, :, :n].view(np.uint16), vsc.view(np.uint16))
    assert int(cache._written.item()) == n
    assert not chain.gave_up()


def test_chain_argument_checks():
    """Inputs the launch cannot take are refused before anything runs."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    L = 2
    cache = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=256, num_q_heads=HQ)
    cache.begin_prefill(100)
    cache.set_prefill_pos(0)
    for l in range(L):
        cache.update(randn((1, H_KV, 100, D), l).cuda(), randn((1, H_KV, 100, D), l + 5).cuda(), l)
    with pytest.raises(RuntimeError):
        ChainedStep(cache, [], [], [], [])  # still prefilling
    cache.finish_prefill(100)
    outs = torch.zeros(L, 1, HQ, 1, D, dtype=torch.float16, device="cuda")
    ks, vs, qs, os_ = _chain_views(outs, L)
    with pytest.raises(ValueError):  # one head stride for every key and value
        ChainedStep(cache, [ks[0], ks[1].contiguous()], vs, qs, os_)
    with pytest.raises(ValueError):  # more layers than the cache holds
        ChainedStep(cache, ks * 2, vs * 2, qs * 2, os_ * 2)
    with pytest.raises(ValueError):
        ChainedStep(cache, ks, vs, qs, [o.float() for o in os_])
    with pytest.raises(NotImplementedError):  # more workgroups than the device holds at once
        ChainedStep(cache, ks, vs, qs, os_, n_parts=100)()
    with pytest.raises(ValueError):
        ChainedStep(cache, ks, vs, qs, os_, dep="none")
    # head h's k from KV head h + 1's rows (the outputs padded by one KV head's rows, so that head
    # 7 reads the padding): layer 0 then reads the previous step's value of layer 1's output,
    # which head h + 1 may overwrite first; only the all-head dependency orders that
    pad = torch.zeros(L, 1, HQ + GQ, 1, D, dtype=torch.float16, device="cuda")
    p_outs = [pad[l, :, :HQ] for l in range(L)]
    p_qs = [p_outs[(l - 1) % L] for l in range(L)]
    p_ks = [pad[(l - 1) % L, :, GQ::GQ] for l in range(L)]
    p_vs = [pad[(l - 1) % L, :, 1::GQ][:, :H_KV] for l in range(L)]
    with pytest.raises(ValueError, match="all-head"):
        ChainedStep(cache, p_ks, p_vs, p_qs, p_outs, dep="head")
    ChainedStep(cache, p_ks, p_vs, p_qs, p_outs, dep="all")
