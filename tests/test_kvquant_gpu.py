"""GPU quantizer parity: bit-exact with the reference's vectors and with the oracle.

Restates the int8 parts of the reference's ``tests/test_kvquant.py`` (226-249) and
``tests/test_kvattn.py::test_pack_matches_quantizer`` (168-175) against the HIP kernels.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kvquant as okq
from tests.helpers import bench_outliers, npy, randn

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
QUANT_FILES = sorted(GOLD.glob("quant_*.npz"))


def _eq16(a: torch.Tensor, b: np.ndarray) -> bool:
    return np.array_equal(npy(a).view(np.uint16), np.asarray(b).view(np.uint16))


@pytest.mark.parametrize("path", QUANT_FILES, ids=[p.stem for p in QUANT_FILES])
def test_gpu_quantizer_matches_reference_vectors(path):
    from nova_amd.kvquant import dequantize_int8, quantize_int8

    z = np.load(path)
    gs, axis = int(z["group"]), str(z["axis"])
    print(f"case {path.stem} shape={z['x'].shape} group={gs} axis={axis}", flush=True)
    x = torch.from_numpy(z["x"]).cuda()
    q, mn, st = quantize_int8(x, gs, axis)
    assert np.array_equal(npy(q), z["q"])
    assert _eq16(mn, z["mins"]) and _eq16(st, z["steps"])
    deq = dequantize_int8(torch.from_numpy(z["q"]).cuda(), torch.from_numpy(z["mins"]).cuda(),
                          torch.from_numpy(z["steps"]).cuda(), gs, axis)
    assert _eq16(deq, z["deq"])


@pytest.mark.parametrize("n", [1, 7, 63, 64, 65, 200, 2048])
def test_token_axis_matches_oracle(n):
    from nova_amd.kvquant import dequantize_int8, quantize_int8

    x = randn((1, 8, n, 128), n, 1.0)
    x = bench_outliers(x, n)
    q, mn, st = quantize_int8(x.cuda(), 64, "token")
    rq, rm, rs = okq.quantize_int8_token(npy(x), 64)
    assert np.array_equal(npy(q), rq)
    assert _eq16(mn, rm) and _eq16(st, rs)
    deq = dequantize_int8(q, mn, st, 64, "token")
    assert _eq16(deq, okq.dequantize_int8_token(rq, rm, rs, 64))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_other_input_dtypes_match_oracle(dtype):
    """The reference upcasts any float input to fp32 first; bf16 and fp32 inputs follow."""
    from nova_amd.kvquant import quantize_int8

    x = (torch.randn(1, 4, 130, 128, generator=torch.Generator().manual_seed(3)) * 2).to(dtype)
    q, mn, st = quantize_int8(x.cuda(), 64, "token")
    rq, rm, rs = okq.quantize_int8_token(x.float().numpy(), 64)
    assert np.array_equal(npy(q), rq)
    assert _eq16(mn, rm) and _eq16(st, rs)


def test_strided_slices_into_cache_match_contiguous():
    """``quantize_int8_into`` writes straight into slices of larger cache buffers."""
    from nova_amd.kvquant import quantize_int8, quantize_int8_into

    src = randn((1, 8, 300, 128), 11).cuda()
    qbuf = torch.full((1, 8, 512, 128), 7, dtype=torch.uint8, device="cuda")
    mbuf = torch.zeros((1, 8, 8, 128), dtype=torch.float16, device="cuda")
    sbuf = torch.zeros_like(mbuf)
    quantize_int8_into(src[:, :, :256], 64, qbuf[:, :, :256], mbuf[:, :, :4], sbuf[:, :, :4])
    q, mn, st = quantize_int8(src[:, :, :256].contiguous(), 64, "token")
    assert torch.equal(qbuf[:, :, :256], q)
    assert torch.equal(mbuf[:, :, :4], mn) and torch.equal(sbuf[:, :, :4], st)
    assert (qbuf[:, :, 256:] == 7).all() and not mbuf[:, :, 4:].any()


def test_constant_and_shapes():
    """``tests/test_kvquant.py:243-249``: constant tensors round-trip exactly, shapes return."""
    from nova_amd.kvquant import dequantize_int8, quantize_int8

    const = torch.full((1, 2, 8, 128), 3.5, dtype=torch.float16, device="cuda")
    for axis, gs in (("channel", 32), ("token", 4)):
        q, mins, steps = quantize_int8(const, gs, axis)
        assert q.shape == const.shape
        assert torch.equal(dequantize_int8(q, mins, steps, gs, axis), const)


def test_error_bounds_against_int4_like_channel_axis():
    """``tests/test_kvquant.py:226-240`` (int8 half): token-axis rulers beat channel-axis
    ones under a channel outlier, and the relative error stays below 0.02."""
    from nova_amd.kvquant import roundtrip_int8

    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, 2, 256, 128, generator=g, dtype=torch.float16)
    x[:, :, :, 7] *= 40
    xc = x.cuda()
    e_chan = (roundtrip_int8(xc, 32, "channel").float() - xc.float()).norm() / xc.float().norm()
    e_tok = (roundtrip_int8(xc, 64, "token").float() - xc.float()).norm() / xc.float().norm()
    assert float(e_chan) < 0.02
    assert float(e_tok) <= float(e_chan)


def test_pack_matches_quantizer():
    from nova_amd.kvattn import GROUP_T, pack_int8_kv
    from nova_amd.kvquant import quantize_int8

    k = randn((1, 8, 200, 128), 5).cuda()
    v = randn((1, 8, 200, 128), 6).cuda()
    kq, kmn, kst, vq, vmn, vst = pack_int8_kv(k, v)
    for got, want in zip((kq, kmn, kst), quantize_int8(k, GROUP_T, "token")):
        assert torch.equal(got, want.contiguous())
    for got, want in zip((vq, vmn, vst), quantize_int8(v, GROUP_T, "token")):
        assert torch.equal(got, want.contiguous())


def test_full_size_prefill_quantize_properties():
    """A 32768-token, 8-head prefill: codes bit-exact with the oracle, and every
    non-degenerate group holds both a 0 and a 255 code."""
    from nova_amd.kvquant import quantize_int8

    x = bench_outliers(randn((1, 8, 32768, 128), 42, 1.0), 43)
    q, mn, st = quantize_int8(x.cuda(), 64, "token")
    rq, rm, rs = okq.quantize_int8_token(npy(x), 64)
    assert np.array_equal(npy(q), rq)
    assert _eq16(mn, rm) and _eq16(st, rs)
    qg = q.view(1, 8, 512, 64, 128)
    assert int(qg.amin(dim=3).max()) == 0 and int(qg.amax(dim=3).min()) == 255
