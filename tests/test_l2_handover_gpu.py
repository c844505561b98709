"""GPU tests of the XCD-local hand-over (``nkv_l2_handover``): the probe of the device's dispatch
of workgroups to XCDs, and the decode launches with the hand-over on (the default after
``_lib.load()``) and off (every partial and forwarded word written through to memory), which must
give bit-identical state and outputs: the store kind changes where a word waits, not its value or
the order of any sum."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import stream as ostream
from tests.helpers import D, H_KV, HQ, assert_ulp_or_abs, npy, randn
from tests.test_chain_gpu import GQ, _assert_state, _chain_views, _prefill_t64

pytestmark = pytest.mark.gpu


@pytest.fixture
def lib():
    from nova_amd import _lib

    _lib.load()
    yield _lib
    _lib.l2_handover(True)  # every test leaves the default on


def test_probe_finds_the_dealing_rule(lib):
    """The probe turns the hand-over on with the device's XCD count (a power of two; 8 on an
    MI355X in its single-partition mode), and off on request."""
    n = lib.l2_handover(True)
    print(f"case l2 probe: {n} XCDs", flush=True)
    assert n in (1, 2, 4, 8)
    assert lib.l2_handover(False) == 0
    assert lib.l2_handover(True) == n


def _assert_same_state(a, b):
    for nm in ("kq", "vq", "kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
        for l, (x, y) in enumerate(zip(getattr(a, nm), getattr(b, nm))):
            assert torch.equal(x, y), f"{nm}[{l}]"
    for nm in ("pos", "_written", "_qlen", "_pg"):
        assert torch.equal(getattr(a, nm), getattr(b, nm)), nm


def _run_chain(lib, on: bool, dep: str, steps: int):
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    lib.l2_handover(on)
    L, n0, cap = 3, 1750, 2048
    cache = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    _prefill_t64(cache, L, n0, seed=70)
    outs = randn((L, 1, HQ, 1, D), 71, scale=0.5).cuda()
    chain = ChainedStep(cache, *_chain_views(outs, L), n_parts=3, dep=dep)
    got = []
    for _ in range(steps):
        chain()
        got.append(npy(outs))
        cache.pos.add_(1)
    chain.check()
    return cache, got


@pytest.mark.parametrize("dep", ["all", "head"])
def test_chain_on_equals_off(lib, dep):
    """The chained step (3 layers, 1750-token prefill over 3 parts, 40 steps across the group
    boundaries at 1792): hand-over on and off give the same outputs and cache state, bit for bit."""
    print(f"case l2 chain on/off dep={dep}", flush=True)
    c_on, o_on = _run_chain(lib, True, dep, 40)
    c_off, o_off = _run_chain(lib, False, dep, 40)
    for s, (a, b) in enumerate(zip(o_on, o_off)):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"step {s}: outputs differ"
    _assert_same_state(c_on, c_off)


def test_chain_through_memory_against_oracle(lib):
    """With the hand-over off, the chained step against the oracle on every layer's own inputs
    (the path every device that was never probed takes)."""
    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache

    print("case l2 off: chain vs oracle", flush=True)
    lib.l2_handover(False)
    L, n0, steps, cap = 3, 250, 72, 512
    cache = KVInt8Cache(num_slots=L, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    ref = ostream.StreamCache(L, H_KV, D, cap, HQ)
    _prefill_t64(cache, L, n0, seed=80, oracle=ref)
    outs = randn((L, 1, HQ, 1, D), 81, scale=0.5).cuda()
    chain = ChainedStep(cache, *_chain_views(outs, L), n_parts=3, dep="all")
    for s in range(steps):
        prev = npy(outs)
        chain()
        got = npy(outs)
        for l in range(L):
            q = (prev if l == 0 else got)[(l - 1) % L][0, :, 0]
            ref.update(q[0::GQ, None], q[1::GQ, None], l)
            assert_ulp_or_abs(got[l][0, :, 0], ref.attend_exact(q, l), 4.0, 1e-3, f"step {s} layer {l}")
        cache.pos.add_(1)
        ref.pos += 1
    _assert_state(cache, ref, L)
    chain.check()


def _run_steps(lib, on: bool, steps: int):
    from nova_amd.kvattn import KVInt8Cache

    lib.l2_handover(on)
    n0, cap = 4000, 4200
    cache = KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    _prefill_t64(cache, 1, n0, seed=90)
    outs = []
    for s in range(steps):
        k = randn((1, H_KV, 1, D), 1000 + s).cuda()
        v = randn((1, H_KV, 1, D), 2000 + s).cuda()
        q = randn((1, HQ, 1, D), 3000 + s, scale=0.3).cuda()
        outs.append(npy(cache.update_attend(k, v, q, 0)))
        cache.pos.add_(1)
    return cache, outs


def test_fused_step_on_equals_off(lib):
    """The per-layer fused step (append, prefix, last-workgroup tail; 4000-token prefill, 100
    steps across the group boundaries at 4032 and 4096): on and off bit-identical."""
    print("case l2 fused step on/off", flush=True)
    c_on, o_on = _run_steps(lib, True, 100)
    c_off, o_off = _run_steps(lib, False, 100)
    for s, (a, b) in enumerate(zip(o_on, o_off)):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"step {s}: outputs differ"
    _assert_same_state(c_on, c_off)


def test_clock_probe_reads_every_xcd(lib):
    """``nkv_clock_probe`` (measurement only): 64 one-wave workgroups dealt over the device's XCDs,
    each with a core clock (core counter over the 100 MHz real-time counter) between the
    device's idle floor and its 2.4 GHz maximum."""
    dev = torch.device("cuda:0")
    n = 64
    buf = torch.zeros(3 * n, dtype=torch.int64, device=dev)
    lib.call("nkv_clock_probe", buf.data_ptr(), n, 20000, lib.stream_ptr(dev))
    torch.cuda.synchronize()
    w = buf.view(n, 3).cpu()
    assert (w[:, 1] > 0).all() and (w[:, 2] > 0).all()
    mhz = 100.0 * w[:, 1].double() / w[:, 2].double()
    assert ((mhz > 50) & (mhz < 2600)).all(), mhz
    n_xcd = len(set(w[:, 0].tolist()))
    assert n_xcd >= 1 and n % n_xcd == 0
