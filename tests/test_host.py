"""Host-side logic that needs no GPU: capacity buckets, the additive mask row, byte accounting."""

from __future__ import annotations

from types import SimpleNamespace

import torch

from oracle import decode as odec
from oracle import kvquant as okq


def test_bucket_for_boundaries():
    """``tests/test_decode_mask_bucket.py:29-37``."""
    from nova_amd.decode import BUCKETS, bucket_for

    assert BUCKETS == odec.BUCKETS
    for n in (1, 2070, 2071, 8192, 16384 + 64, 32768 + 256, 65536, 70000):
        assert bucket_for(n) == odec.bucket_for(n)
    assert bucket_for(1) == 2070 and bucket_for(2071) == 4096 and bucket_for(70000) == 70000


def test_mask_row_matches_table_bitwise():
    """``_mask_row(pos)`` equals row ``pos`` of ``_build_mask_table`` including the min
    values (``tests/test_decode_mask_bucket.py:40-57``), and the oracle's row."""
    from nova_amd.decode import GraphDecoder

    max_len = 64
    table = GraphDecoder._build_mask_table(max_len, torch.float16, "cpu")
    fake = SimpleNamespace(max_len=max_len, _arange=torch.arange(max_len, dtype=torch.long),
                           _zero=torch.zeros((), dtype=torch.float16),
                           _ninf=torch.full((), torch.finfo(torch.float16).min, dtype=torch.float16))
    for pos in (0, 1, 7, 63):
        row = GraphDecoder._mask_row(fake, torch.tensor([pos]))
        assert row.shape == (1, 1, 1, max_len)
        assert torch.equal(row.reshape(max_len), table[pos])
        assert torch.equal(row.reshape(max_len), torch.from_numpy(odec.mask_row(pos, max_len)))


def test_bytes_per_token_int8():
    from nova_amd.kvquant import bytes_per_token

    a = bytes_per_token(36, 8, 128, bits=8)
    b = bytes_per_token(36, 8, 128, bits=8, k_axis="token", token_group=64)
    assert a == okq.bytes_per_token_int8(36, 8, 128)
    assert b == okq.bytes_per_token_int8(36, 8, 128, k_axis="token", token_group=64)
    assert 1.85 <= b["ratio"] <= 1.95


def _tiny_model(intermediate: int = 96):
    from nova_amd.skeleton import SkeletonConfig, SkeletonForCausalLM

    cfg = SkeletonConfig(num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                         hidden_size=64, intermediate_size=intermediate, vocab_size=50)
    return cfg, SkeletonForCausalLM(cfg, seed=3).eval()


def test_skeleton_mlp_is_leanmlp_and_layer_is_pre_norm_residual():
    """``SkeletonMLP`` computes ``down(silu(gate(x)) * up(x))`` (``LeanMLP``, src/nova/layers.py:
    173-174) and a layer adds attention and MLP to the residual stream after their RMSNorms
    (``LeanDecoderLayer.forward``, layers.py:195-218); the MLP is absent with intermediate_size 0."""
    import torch.nn.functional as F

    cfg, model = _tiny_model()
    layer = model.model.layers[0]
    x = torch.randn(1, 3, cfg.hidden_size, generator=torch.Generator().manual_seed(0))
    m = layer.mlp
    want = (F.silu(x @ m.gate_proj.weight.T) * (x @ m.up_proj.weight.T)) @ m.down_proj.weight.T
    assert torch.allclose(m(x), want, atol=1e-5)
    _, no_mlp = _tiny_model(0)
    assert no_mlp.model.layers[0].mlp is None and no_mlp.model.layers[0].post_norm is None


def test_skeleton_stacked_weights_are_views_of_one_buffer():
    """``stack_weights`` puts q/k/v and gate/up into single row-stacked weights whose slices
    the Linear layers keep using, so the torch path and the kernel path read the same bytes."""
    _, model = _tiny_model()
    layer = model.model.layers[1]
    before = [t.clone() for t in (layer.attn.q_proj.weight, layer.attn.k_proj.weight, layer.attn.v_proj.weight,
                                  layer.mlp.gate_proj.weight, layer.mlp.up_proj.weight)]
    layer.stack_weights()
    qkv, gu = layer.w_qkv, layer.w_gate_up
    assert torch.equal(qkv, torch.cat(before[:3])) and torch.equal(gu, torch.cat(before[3:]))
    assert layer.attn.k_proj.weight.data_ptr() == qkv[before[0].shape[0]:].data_ptr()
    assert layer.mlp.up_proj.weight.data_ptr() == gu[before[3].shape[0]:].data_ptr()


def test_kernel_mode_needs_an_fp16_gpu_model():
    _, model = _tiny_model()
    import pytest

    with pytest.raises(ValueError, match="fp16 on the GPU"):
        model.use_decode_kernels(True)
    assert model.model.decode_kernels is False


def test_gemv_wrappers_refuse_cpu_tensors():
    """The projection wrappers check their tensors before any library call (no fallback)."""
    import pytest

    from nova_amd import gemv as G

    x = torch.zeros(64, dtype=torch.float16)
    w = torch.zeros(8, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="CUDA"):
        G.rms_gemv(x, w)
    with pytest.raises(ValueError, match="CUDA"):
        G.swiglu_gemv(x, torch.zeros(16, 64, dtype=torch.float16))
    with pytest.raises(ValueError):
        G.qk_norm_rope_(torch.zeros(6 * 128, dtype=torch.float16), 4, 1, x, x, 1e-6, torch.zeros(64), torch.zeros(1))


def test_capture_pool_choices():
    """``capture(pool=...)`` takes the reference's choices (src/nova/decode.py:379-442): "off" and
    None mean no pool, "auto"/"shared" the shared pool (registered), anything else passes through;
    other strings are refused."""
    import pytest

    from nova_amd import decode as dec

    assert dec.resolve_pool("off") == (None, False)
    assert dec.resolve_pool(None) == (None, False)
    handle = object()
    assert dec.resolve_pool(handle) == (handle, False)
    with pytest.raises(ValueError, match="pool"):
        dec.resolve_pool("bogus")
    # the shared-pool bookkeeping, with a stand-in for torch's handle
    calls = []
    reg = dec._PoolRegistry()
    orig = torch.cuda.graph_pool_handle
    torch.cuda.graph_pool_handle = lambda: calls.append(1) or ("pool", len(calls))
    try:
        a = reg.pool(fresh_if_idle=True)
        assert reg.pool(fresh_if_idle=False) == a          # "shared": the same pool
        b = reg.pool(fresh_if_idle=True)                    # "auto", no live user: a fresh pool
        assert b != a

        class G:  # a graph stand-in (weakly referenced)
            pass

        g = G()
        reg.register(g)
        assert reg.pool(fresh_if_idle=True) == b            # a live user keeps the pool
        del g
        assert reg.pool(fresh_if_idle=True) != b            # its graph is gone: fresh again
    finally:
        torch.cuda.graph_pool_handle = orig


def test_mask_table_rows():
    from nova_amd.decode import GraphDecoder

    t = GraphDecoder._build_mask_table(5, torch.float16, "cpu")
    lo = torch.finfo(torch.float16).min
    for p in range(5):
        assert all(float(t[p, j]) == (0.0 if j <= p else lo) for j in range(5))


def test_page_pool_guards():
    """Host bookkeeping of the paged cache: reservations grow from group 0, a release returns every
    page, a step past the reserved pages is refused (before any kernel could write through a page
    table entry the sequence does not own), and the pool refuses to overcommit."""
    import pytest

    from nova_amd.paged import GT, PagePool

    pool = PagePool(num_pages=10, max_seqs=3, max_pages_per_seq=6)
    assert pool.reserve(0, 65) == [(0, 0), (1, 1)]           # groups 0 and 1, pages from the free list
    assert pool.reserve(0, 100) == []                         # already covered
    assert [g for g, _ in pool.reserve(1, 3 * GT)] == [0, 1, 2]
    pool.set_length(0, 65)
    pool.advance(1, 63)                                       # tokens 65 .. 127 stay in page 1
    with pytest.raises(RuntimeError, match="reserve"):
        pool.advance(1, 1)                                    # token 128 would need group 2
    assert pool.length[0] == 128
    with pytest.raises(RuntimeError, match="reserved"):
        pool.set_length(1, 3 * GT + 1)
    with pytest.raises(RuntimeError, match="exhausted"):
        pool.reserve(2, 6 * GT)                               # 6 pages, 5 free
    with pytest.raises(ValueError, match="max_pages_per_seq"):
        pool.reserve(2, 7 * GT)
    owned0 = list(pool.owned[0])
    pool.release(0)
    assert pool.owned[0] == [] and pool.length[0] == 0 and set(owned0) <= set(pool.free)
    assert sorted(pool.free + pool.owned[1]) == list(range(10))
    with pytest.raises(ValueError):
        pool.reserve(3, 1)                                    # no such sequence


def test_plan_parts_bounds():
    """The paged work plan gives every sequence at least one and at most 256 parts, in proportion
    to its groups, and numbers the units consecutively per sequence."""
    from nova_amd.paged import MAX_PARTS_PER_SEQ, plan_parts

    wg, sp = plan_parts([4566, 13658, 10122, 8480, 9727, 12101, 7956, 10569], 32)
    assert len(sp) == 16 and sum(sp[1::2]) == len(wg)
    for b in range(8):
        first, n = sp[2 * b], sp[2 * b + 1]
        assert n >= 1 and [w >> 16 for w in wg[first:first + n]] == [b] * n
        assert [w & 0xffff for w in wg[first:first + n]] == list(range(n))
    # a long sequence beside short ones still gets at most MAX_PARTS_PER_SEQ parts
    wg, sp = plan_parts([1 << 20, 64, 64], 4096)
    assert sp[1] == MAX_PARTS_PER_SEQ and sp[3] >= 1 and sp[5] >= 1
