"""GPU parity of the streamed (64-multiple chunked) prefill of ``KVInt8Cache``.

The reference keeps the whole prompt in fp16 staging and quantizes it at the end, and
names chunked quantization in multiples of 64 as the fix
(``reports/kv-int8-streaming-cache.md:126-131``). Two properties pin the streamed form:

- state: every 64-token group is quantized from the same fp16 tokens, so codes, rulers,
  ring and scalars after ``finish_prefill`` equal the staged path's bit for bit (and so do
  the decode steps that follow);
- attention: each chunk attends the int8 history ``[0, off)`` plus itself causally, so its
  output meets the chunked-prefill criterion against ``oracle.attn.chunk_prefill_attend``
  (max-abs <= 2e-3, mean-abs <= 1.5e-4).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from tests.helpers import D, H_KV, HQ, npy, randn

pytestmark = pytest.mark.gpu

LAYERS = 2


def _caches(total, cap_extra=64):
    from nova_amd.kvattn import KVInt8Cache

    mk = lambda: KVInt8Cache(num_slots=LAYERS, num_kv_heads=H_KV, head_dim=D, max_len=total + cap_extra,
                             num_q_heads=HQ)
    return mk(), mk()


def _staged(c, k, v, total):
    c.begin_prefill(total)
    c.set_prefill_pos(0)
    for layer in range(LAYERS):
        c.update(k[layer][:, :, :total], v[layer][:, :, :total], layer)
    c.finish_prefill(total)


def _state(c):
    t = [c.pos, c.first, c._written, c._qlen, c._pg]
    for layer in range(LAYERS):
        t += [c.kq[layer], c.kmn[layer], c.kst[layer], c.vq[layer], c.vmn[layer], c.vst[layer],
              c.tail_k[layer], c.tail_v[layer]]
    return t


def _oracle_chunk(c, layer, q, kch, vch, off):
    pk = [npy(t)[0] for t in (c.kq[layer], c.kmn[layer], c.kst[layer], c.vq[layer], c.vmn[layer], c.vst[layer])]
    return oattn.chunk_prefill_attend(npy(q)[0], *pk, off, npy(kch)[0], npy(vch)[0])


@pytest.mark.parametrize("total,chunk", [(1000, 256), (512, 512), (130, 64), (40, 64), (577, 192)])
def test_streamed_prefill_matches_staged_state_and_oracle(total, chunk):
    print(f"case total={total} chunk={chunk}", flush=True)
    k = [randn((1, H_KV, total, D), 300 + layer, 1.0).cuda() for layer in range(LAYERS)]
    v = [randn((1, H_KV, total, D), 310 + layer, 1.0).cuda() for layer in range(LAYERS)]
    q = [randn((1, HQ, total, D), 320 + layer, 1.0).cuda() for layer in range(LAYERS)]
    staged, streamed = _caches(total)
    _staged(staged, k, v, total)
    streamed.begin_prefill(total, stream_chunk=chunk)
    assert streamed.staging is None and streamed.prefilling
    for off in range(0, total, chunk):
        n = min(chunk, total - off)
        streamed.set_prefill_pos(off)
        for layer in range(LAYERS):
            kch, vch = k[layer][:, :, off:off + n], v[layer][:, :, off:off + n]
            streamed.update(kch, vch, layer)
            got = streamed.attend_prefill(q[layer][:, :, off:off + n], layer)
            # the staged cache holds the same groups [0, off) (bit-exact, checked below)
            want = _oracle_chunk(staged, layer, q[layer][:, :, off:off + n], kch, vch, off)
            err = np.abs(npy(got)[0].astype(np.float64) - want)
            assert err.max() <= 2e-3, f"off={off} layer={layer}: max abs {err.max():.2e}"
            assert err.mean() <= 1.5e-4, f"off={off} layer={layer}: mean abs {err.mean():.2e}"
    streamed.finish_prefill(total)
    assert not streamed.prefilling
    for i, (a, b) in enumerate(zip(_state(streamed), _state(staged))):
        assert torch.equal(a, b), f"state tensor {i}"
    # the decode steps that follow are identical too
    for step in range(3):
        kn = randn((1, H_KV, 1, D), 400 + step).cuda()
        vn = randn((1, H_KV, 1, D), 410 + step).cuda()
        qn = randn((1, HQ, 1, D), 420 + step).cuda()
        for layer in range(LAYERS):
            a = streamed.update_attend(kn, vn, qn, layer).clone()
            b = staged.update_attend(kn, vn, qn, layer)
            assert torch.equal(a, b), (step, layer)
        for c in (streamed, staged):
            c.pos.add_(1)


def test_streamed_prefill_argument_errors():
    _, c = _caches(256)
    k = randn((1, H_KV, 256, D), 1).cuda()
    with pytest.raises(ValueError, match="64"):
        c.begin_prefill(256, stream_chunk=100)
    c.begin_prefill(256, stream_chunk=128)
    c.set_prefill_pos(0)
    with pytest.raises(ValueError, match="stream_chunk"):
        c.update(k[:, :, :192], k[:, :, :192], 0)
    c.update(k[:, :, :100], k[:, :, :100], 0)
    # the next chunk must start where this one ended ...
    with pytest.raises(ValueError):
        c.set_prefill_pos(128)
    c.set_prefill_pos(100)
    # ... and only the last chunk may end off a group boundary
    with pytest.raises(ValueError, match="64"):
        c.update(k[:, :, 100:164], k[:, :, 100:164], 0)
    with pytest.raises(RuntimeError):
        c.attend_prefill(randn((1, HQ, 64, D), 2).cuda(), 0)
    with pytest.raises(ValueError):
        c.finish_prefill(256)


def test_graph_decoder_streamed_prefill():
    """``GraphDecoder.prefill(chunk=128)`` through a 3-layer random-weight model: layer 0's
    int8 cache equals the staged prefill's bit for bit (its K/V do not depend on attention),
    deeper layers see K/V computed after an int8-history attention, so they and the logits
    only stay close; the captured decode steps that follow run and stay close as well."""
    from nova_amd.decode import GraphDecoder
    from nova_amd.skeleton import SkeletonConfig, SkeletonForCausalLM

    cfg = SkeletonConfig(num_hidden_layers=3, hidden_size=1024, vocab_size=1024, intermediate_size=0)
    model = SkeletonForCausalLM(cfg, seed=0).half().cuda().eval()
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 1024, (1, 333), generator=g).cuda()
    decs, logits = [], []
    for chunk in (0, 128):
        dec = GraphDecoder(model, max_len=512, quant="int8")
        logits.append(dec.prefill(ids, chunk=chunk).float())
        decs.append(dec)
    a, b = decs
    assert int(a.cache.pos.item()) == int(b.cache.pos.item()) == 333
    for nm in ("kq", "kmn", "kst", "vq", "vmn", "vst", "tail_k", "tail_v"):
        assert torch.equal(getattr(a.cache, nm)[0], getattr(b.cache, nm)[0]), nm
    for layer in range(1, cfg.num_hidden_layers):
        x, y = a.cache.tail_k[layer].float(), b.cache.tail_k[layer].float()
        assert (x - y).norm() / x.norm() < 2e-2, layer
    rels = [float((logits[0] - logits[1]).norm() / logits[0].norm())]
    b.input_ids.copy_(a.input_ids)  # start both from the same token
    for dec in decs:
        dec.capture(warmup=2)
    for _ in range(4):
        for dec in decs:
            dec.step()
        torch.cuda.synchronize()
        assert torch.isfinite(a.logits).all() and torch.isfinite(b.logits).all()
        rels.append(float((a.logits.float() - b.logits.float()).norm() / a.logits.float().norm()))
        b.input_ids.copy_(a.input_ids)
    print(f"relative logit differences streamed vs staged: {[f'{r:.2e}' for r in rels]}", flush=True)
    assert max(rels) < 1e-2, rels
