"""End-to-end graph decode through the int8 cache — restates the reference's
``tests/test_graph_decode_int8.py`` on a random-weight attention-only decoder with the
Qwen3-4B attention geometry (the reference's tests load the real checkpoint, which is
not available offline)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_LEN = 256


@pytest.fixture(scope="module")
def model():
    from nova_amd.skeleton import SkeletonConfig, SkeletonForCausalLM

    cfg = SkeletonConfig(num_hidden_layers=4, hidden_size=1024, vocab_size=1024, intermediate_size=0)
    return SkeletonForCausalLM(cfg, seed=0).half().cuda().eval()


@pytest.fixture(scope="module")
def prompt_ids():
    g = torch.Generator().manual_seed(0)
    return torch.randint(0, 1024, (1, 77), generator=g).cuda()


@pytest.mark.parametrize("quant", ["off", "int8"])
def test_capture_replay_matches_eager(model, prompt_ids, quant):
    """A replay of the captured step equals the eager step's logits bit for bit."""
    from nova_amd.decode import GraphDecoder

    dec = GraphDecoder(model, max_len=MAX_LEN, quant=quant)
    dec.prefill(prompt_ids)
    pos0 = int(dec.cache.pos.item())
    ids0 = dec.input_ids.clone()
    saved = dec._save_int8_state()
    with torch.inference_mode():
        eager = dec._body().clone()
    dec.cache.pos.fill_(pos0)
    dec.input_ids.copy_(ids0)
    dec._restore_int8_state(saved)
    if quant == "int8":
        dec.cache.refresh_scalars()
    dec.capture(warmup=2)
    dec.step()
    torch.cuda.synchronize()
    assert torch.equal(dec.logits, eager)


def test_int8_decode_agrees_with_fp16_on_tokens(model, prompt_ids):
    """Both caches generate 8 greedy tokens; at least 6 agree (int8 is lossy; decode is
    autoregressive, ``tests/test_graph_decode_int8.py:56-70``), and the first step's
    logits stay close."""
    from nova_amd.decode import GraphDecoder

    outs, logits = {}, {}
    for quant in ("off", "int8"):
        dec = GraphDecoder(model, max_len=MAX_LEN, quant=quant)
        first = dec.prefill(prompt_ids)
        dec.capture(warmup=2)
        toks = [int(dec.input_ids.item())]
        for i in range(7):
            lg = dec.step()
            if i == 0:
                logits[quant] = lg.float().clone()
            toks.append(int(dec.input_ids.item()))
        outs[quant] = toks
        assert torch.isfinite(first).all()
    agree = sum(a == b for a, b in zip(outs["off"], outs["int8"]))
    assert agree >= 6, outs
    rel = (logits["int8"] - logits["off"]).norm() / logits["off"].norm()
    assert float(rel) < 0.05, float(rel)


def test_generate_crosses_group_boundaries(model):
    """Decode 140 tokens from a 60-token prompt: the int8 prefix grows through three
    group boundaries inside one captured graph; the scalars track the position."""
    from nova_amd.decode import GraphDecoder

    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 1024, (1, 60), generator=g).cuda()
    dec = GraphDecoder(model, max_len=MAX_LEN, quant="int8")
    out = dec.generate(ids, 140)
    torch.cuda.synchronize()
    assert out.shape == (1, 140)
    pos = int(dec.cache.pos.item())
    assert pos == 60 + 139
    assert int(dec.cache._written.item()) == pos
    assert int(dec.cache._qlen.item()) == pos // 64 * 64


def test_int8_cache_is_smaller(model):
    from nova_amd.decode import GraphDecoder

    off = GraphDecoder(model, max_len=2048, quant="off")
    i8 = GraphDecoder(model, max_len=2048, quant="int8")
    ratio = i8.cache.nbytes() / off.cache.nbytes()
    assert 0.4 < ratio < 0.6, ratio


def test_int8_grow_is_refused(model):
    from nova_amd.decode import GraphDecoder

    dec = GraphDecoder(model, max_len=MAX_LEN, quant="int8")
    with pytest.raises(NotImplementedError):
        dec.grow(MAX_LEN * 2)
    with pytest.raises(ValueError, match="quant"):
        GraphDecoder(model, max_len=MAX_LEN, quant="int4")
