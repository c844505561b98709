"""GPU parity of the fused attention-block step (``nkv_decode_step_qkv_t64``,
``KVInt8Cache.update_attend_qkv`` / ``update_attend_block``): the input RMSNorm and stacked q/k/v
projection, the q/k head norms with the rotary embedding, the append + attention of the token and
(``update_attend_block``) the output projection with the residual add, in one launch.

The step computes every value exactly as the separate launches do (``nkv_gemv`` with the input
norm, ``nkv_qk_norm_rope``, ``nkv_decode_step_t64``: the same input chunks per thread, the same
reductions and summation orders, the same fp16 roundings), so it is checked against them bit for
bit: the q/k/v vectors it used, the attention output and the whole cache state, over steps that
cross group boundaries, at a short context (one streaming workgroup per head), a mid one and 32k.
Those separate launches are themselves checked against float64 references and the oracle
(``tests/test_gemv_gpu.py``, ``tests/test_kvattn_stream_gpu.py``).
"""

from __future__ import annotations

import pytest
import torch

from tests.helpers import D, H_KV, HQ
from tests.test_chain_gpu import _prefill_t64

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cuda").manual_seed(seed)


def _params(hidden: int, seed: int):
    rows = (HQ + 2 * H_KV) * D
    w = (torch.randn(rows, hidden, generator=_gen(seed), device="cuda") * hidden ** -0.5).half()
    xg = (1.0 + 0.1 * torch.randn(hidden, generator=_gen(seed + 1), device="cuda")).half()
    qg = (1.0 + 0.1 * torch.randn(D, generator=_gen(seed + 2), device="cuda")).half()
    kg = (1.0 + 0.1 * torch.randn(D, generator=_gen(seed + 3), device="cuda")).half()
    inv = (1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).cuda()
    return w, xg, qg, kg, inv


def _x(hidden: int, seed: int) -> torch.Tensor:
    return torch.randn(hidden, generator=_gen(seed), device="cuda").half()


def _separate(cache, x, w, xg, qg, kg, inv):
    """The same layer step as separate launches: qkv GEMV, head norms + RoPE, fused decode step."""
    from nova_amd import gemv as G

    qkv = G.rms_gemv(x, w, xg, EPS)
    G.qk_norm_rope_(qkv, HQ, H_KV, qg, kg, EPS, inv, cache.pos)
    q = qkv[:HQ * D].view(1, HQ, 1, D)
    k = qkv[HQ * D:(HQ + H_KV) * D].view(1, H_KV, 1, D)
    v = qkv[(HQ + H_KV) * D:].view(1, H_KV, 1, D)
    return qkv, cache.update_attend(k, v, q, 0).clone()


def _assert_same_state(a, b):
    for nm in ("kq", "vq", "kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
        assert torch.equal(getattr(a, nm)[0], getattr(b, nm)[0]), nm
    for nm in ("pos", "_written", "_qlen", "_pg"):
        assert torch.equal(getattr(a, nm), getattr(b, nm)), nm


@pytest.mark.parametrize("hidden,n0,steps,cap", [(2560, 4000, 100, 4200), (2560, 200, 70, 512), (1024, 1990, 60, 2112),
                                                 (2560, 32765, 4, 32832)])
def test_fused_step_equals_separate_launches(hidden, n0, steps, cap):
    """Twin caches from one prefill; each step, the same x through the fused step and through the
    separate launches: q/k/v (qkv_out), the output and, at the end, the cache state bit for bit."""
    from nova_amd.kvattn import KVInt8Cache

    print(f"case qkv step hidden={hidden} n0={n0} steps={steps} cap={cap}", flush=True)
    w, xg, qg, kg, inv = _params(hidden, 10)
    fused = KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    sep = KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    _prefill_t64(fused, 1, n0, seed=20)
    _prefill_t64(sep, 1, n0, seed=20)
    qkv_out = torch.empty((HQ + 2 * H_KV) * D, dtype=torch.float16, device="cuda")
    for s in range(steps):
        x = _x(hidden, 100 + s)
        qkv, want = _separate(sep, x, w, xg, qg, kg, inv)
        got = fused.update_attend_qkv(x, w, xg, EPS, qg, kg, EPS, inv, 0, qkv_out=qkv_out)
        torch.cuda.synchronize()
        assert torch.equal(qkv_out, qkv), f"step {s}: q/k/v differ from the separate launches"
        assert torch.isfinite(got.float()).all(), f"step {s}: non-finite output"
        assert torch.equal(got, want), f"step {s}: output differs from the separate launches"
        fused.pos.add_(1)
        sep.pos.add_(1)
    _assert_same_state(fused, sep)


def _w_o(hidden: int, seed: int) -> torch.Tensor:
    return (torch.randn(hidden, HQ * D, generator=_gen(seed), device="cuda") * (HQ * D) ** -0.5).half()


@pytest.mark.parametrize("hidden,n0,steps,cap", [(2560, 4000, 60, 4200), (2560, 200, 40, 512), (1024, 1990, 40, 2112),
                                                 (2560, 32765, 4, 32832)])
def test_block_with_o_proj_equals_separate_launches(hidden, n0, steps, cap):
    """The attention block with its output projection (``update_attend_block``): h1 = x + W_o o,
    the attention output o and the cache state, bit for bit the separate launches' (the GEMV
    computes o_proj with the residual), over steps; every other step updates x in place."""
    from nova_amd import gemv as G
    from nova_amd.kvattn import KVInt8Cache

    print(f"case attention block + o_proj hidden={hidden} n0={n0} steps={steps} cap={cap}", flush=True)
    w, xg, qg, kg, inv = _params(hidden, 80)
    w_o = _w_o(hidden, 81)
    fused = KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    sep = KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ)
    _prefill_t64(fused, 1, n0, seed=82)
    _prefill_t64(sep, 1, n0, seed=82)
    qkv_out = torch.empty((HQ + 2 * H_KV) * D, dtype=torch.float16, device="cuda")
    o_f = torch.empty(1, HQ, 1, D, dtype=torch.float16, device="cuda")
    for s in range(steps):
        x = _x(hidden, 300 + s)
        qkv, o_s = _separate(sep, x, w, xg, qg, kg, inv)
        want = G.rms_gemv(o_s.reshape(-1), w_o, residual=x)
        xin = x.clone()
        h1 = fused.update_attend_block(xin, w, xg, EPS, qg, kg, EPS, inv, w_o, 0, out=o_f, qkv_out=qkv_out,
                                       h1_out=xin if s % 2 else None)
        torch.cuda.synchronize()
        assert torch.equal(qkv_out, qkv), f"step {s}: q/k/v differ"
        assert torch.equal(o_f, o_s), f"step {s}: attention output differs"
        assert torch.isfinite(h1.float()).all(), f"step {s}: non-finite h1"
        assert torch.equal(h1, want), f"step {s}: h1 differs from the separate launches"
        if s % 2:
            assert h1.data_ptr() == xin.data_ptr()
        fused.pos.add_(1)
        sep.pos.add_(1)
    _assert_same_state(fused, sep)


def test_block_with_o_proj_graph_replay_equals_eager():
    """The block with o_proj captured once and replayed (x from a fixed buffer, h1 into a buffer
    of its own) equals eager calls on a twin cache, bit for bit."""
    from nova_amd.kvattn import KVInt8Cache

    print("case attention block + o_proj graph replay", flush=True)
    hidden, n0, cap = 2560, 3000, 3200
    w, xg, qg, kg, inv = _params(hidden, 90)
    w_o = _w_o(hidden, 91)
    caches = [KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ) for _ in range(2)]
    for c in caches:
        _prefill_t64(c, 1, n0, seed=92)
    g_cache, e_cache = caches
    xbuf = _x(hidden, 0)
    h1 = torch.empty(hidden, dtype=torch.float16, device="cuda")
    for c in caches:  # one eager step each (the workspace grows outside the capture)
        c.update_attend_block(xbuf, w, xg, EPS, qg, kg, EPS, inv, w_o, 0, h1_out=h1)
        c.pos.add_(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            g_cache.update_attend_block(xbuf, w, xg, EPS, qg, kg, EPS, inv, w_o, 0, h1_out=h1)
            g_cache.pos.add_(1)
    torch.cuda.current_stream().wait_stream(stream)
    for s in range(40):
        x = _x(hidden, 400 + s)
        xbuf.copy_(x)
        graph.replay()
        want = e_cache.update_attend_block(x, w, xg, EPS, qg, kg, EPS, inv, w_o, 0)
        e_cache.pos.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(h1, want), f"step {s}: replay differs from eager"
    _assert_same_state(g_cache, e_cache)


def test_block_with_o_proj_argument_checks():
    from nova_amd.kvattn import KVInt8Cache

    hidden = 2560
    w, xg, qg, kg, inv = _params(hidden, 95)
    c = KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=512, num_q_heads=HQ)
    _prefill_t64(c, 1, 100, seed=96)
    x = _x(hidden, 1)
    with pytest.raises(ValueError):  # w_o of the wrong shape
        c.update_attend_block(x, w, xg, EPS, qg, kg, EPS, inv, _w_o(hidden, 97)[:, :2048].contiguous(), 0)
    with pytest.raises(ValueError):  # h1_out of the wrong size
        c.update_attend_block(x, w, xg, EPS, qg, kg, EPS, inv, _w_o(hidden, 98), 0,
                              h1_out=torch.empty(100, dtype=torch.float16, device="cuda"))
    o = torch.empty(1, HQ, 1, D, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):  # h1_out overlapping the attention output
        c.update_attend_block(x, w, xg, EPS, qg, kg, EPS, inv, _w_o(hidden, 99), 0, out=o, h1_out=o.view(-1)[:hidden])


def test_fused_step_graph_replay_equals_eager():
    """The fused step captured once (x read from a fixed buffer) and replayed step after step
    equals eager calls on a twin cache, bit for bit."""
    from nova_amd.kvattn import KVInt8Cache

    print("case qkv step graph replay", flush=True)
    hidden, n0, cap = 2560, 3000, 3200
    w, xg, qg, kg, inv = _params(hidden, 30)
    caches = [KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=cap, num_q_heads=HQ) for _ in range(2)]
    for c in caches:
        _prefill_t64(c, 1, n0, seed=40)
    g_cache, e_cache = caches
    xbuf = _x(hidden, 0)
    out = torch.empty(1, HQ, 1, D, dtype=torch.float16, device="cuda")
    for c in caches:  # one eager step each (the workspace grows outside the capture)
        c.update_attend_qkv(xbuf, w, xg, EPS, qg, kg, EPS, inv, 0, out=out)
        c.pos.add_(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            g_cache.update_attend_qkv(xbuf, w, xg, EPS, qg, kg, EPS, inv, 0, out=out)
            g_cache.pos.add_(1)
    torch.cuda.current_stream().wait_stream(stream)
    for s in range(70):
        x = _x(hidden, 200 + s)
        xbuf.copy_(x)
        graph.replay()
        want = e_cache.update_attend_qkv(x, w, xg, EPS, qg, kg, EPS, inv, 0)
        e_cache.pos.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"step {s}: replay differs from eager"
    _assert_same_state(g_cache, e_cache)


def test_fused_step_argument_checks():
    from nova_amd.kvattn import KVInt8Cache

    hidden = 2560
    w, xg, qg, kg, inv = _params(hidden, 50)
    c = KVInt8Cache(num_slots=1, num_kv_heads=H_KV, head_dim=D, max_len=512, num_q_heads=HQ)
    _prefill_t64(c, 1, 100, seed=60)
    x = _x(hidden, 1)
    with pytest.raises(ValueError):
        c.update_attend_qkv(x, w[:, :1024].contiguous(), xg, EPS, qg, kg, EPS, inv, 0)
    with pytest.raises(ValueError):
        c.update_attend_qkv(x, w, xg, EPS, qg, kg, EPS, inv.half(), 0)
    big = 4096
    wb, xgb, *_ = _params(big, 70)
    with pytest.raises(NotImplementedError):  # hidden beyond 3072
        c.update_attend_qkv(_x(big, 2), wb, xgb, EPS, qg, kg, EPS, inv, 0)


def test_decoder_fused_equals_separate():
    """A 3-layer decoder (hidden 2560, the Qwen3-4B head geometry) in kernel mode: the fused
    attention-block launch and the separate launches give the same logits, bit for bit, over
    graph-decoded steps."""
    from nova_amd.decode import GraphDecoder
    from nova_amd.skeleton import SkeletonConfig, SkeletonForCausalLM

    print("case qkv decoder fused vs separate", flush=True)
    cfg = SkeletonConfig(num_hidden_layers=3, hidden_size=2560, intermediate_size=2048, vocab_size=4096)
    model = SkeletonForCausalLM(cfg, seed=0).half().cuda().eval()
    ids = torch.randint(0, cfg.vocab_size, (1, 260), generator=torch.Generator().manual_seed(9)).cuda()
    logits = {}
    for fused in (True, False):
        model.use_decode_kernels(True, fused_qkv=fused)
        dec = GraphDecoder(model, max_len=512, quant="int8")
        dec.prefill(ids)
        dec.capture(warmup=2)
        out = []
        for _ in range(6):
            dec.step()
            out.append(dec.logits.clone())
        torch.cuda.synchronize()
        logits[fused] = out
    model.use_decode_kernels(False)
    for i, (a, b) in enumerate(zip(logits[True], logits[False])):
        assert torch.equal(a, b), f"step {i}: fused and separate logits differ"
