"""GPU parity of the decode-step projection kernels (``nova_amd.gemv``) and of the decoder
that runs on them.

Each kernel is checked against a float64 reference of the same op on the same fp16 inputs,
with the fp16 roundings the op defines (the torch ops of ``nova_amd.skeleton``: RMSNorm output
rounded to fp16, the projection's result rounded to fp16, then the residual add, SwiGLU's
``silu(fp16 g) * fp16 u``). What is left is fp32 summation order and, rarely, the last bit
of the RMSNorm factor (the kernel sums the mean of squares in another order than torch, a few
float ULPs apart, which flips the fp16 rounding of some normalized inputs): every element within 2 fp16 ULP or 1e-4 absolute (GEMVs; with a
residual, ulp(|W x|) + ulp(|y|), since the projection is rounded before the add), 3 ULP or
1e-4 (SwiGLU, whose two fp16 roundings of g and u can each move by one), and for norm + RoPE,
against the skeleton's own torch ops on the GPU, one rounding flip of each of its two terms
plus one of their sum.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.helpers import assert_ulp_or_abs, npy

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cuda").manual_seed(seed)


def _w(out: int, n_in: int, seed: int) -> torch.Tensor:
    return (torch.randn(out, n_in, generator=_gen(seed), device="cuda") * n_in ** -0.5).half()


def _x(n: int, seed: int, scale: float = 1.0) -> torch.Tensor:
    return (torch.randn(n, generator=_gen(seed), device="cuda") * scale).half()


def _rms16(x: torch.Tensor, gamma: torch.Tensor | None) -> torch.Tensor:
    """The op's normalized input: torch's fp16 RMSNorm (the skeleton's ``_rms``)."""
    if gamma is None:
        return x
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).half() * gamma


def _ref_gemv(x, w, gamma, residual):
    y = (w.double() @ _rms16(x, gamma).double()).half()
    if residual is not None:
        y = y + residual
    return y


def _spacing16(a: np.ndarray) -> np.ndarray:
    a16 = np.abs(a).astype(np.float16)
    return np.nextafter(a16, np.float16(np.inf)).astype(np.float64) - a16.astype(np.float64)


def _check(got, want, x, w, gamma, residual, tag):
    """Without a residual: 2 ULP or 1e-4 abs. With one, the projection is rounded to fp16 before
    the add, so when the two nearly cancel the error is set by the projection's magnitude:
    within ulp(|W xn|) + ulp(|y|) (one flip of each rounding) or 1e-4 abs."""
    if residual is None:
        return assert_ulp_or_abs(npy(got), npy(want.float()), 2, 1e-4, tag)
    proj = npy(w.double() @ _rms16(x, gamma).double())
    g, wnt = npy(got).astype(np.float64), npy(want).astype(np.float64)
    diff = np.abs(g - wnt)
    bound = _spacing16(proj) + _spacing16(wnt)
    bad = (diff > bound) & (diff > 1e-4)
    assert int(bad.sum()) == 0, f"{tag}: {int(bad.sum())} elements beyond ulp(|W x|) + ulp(|y|) and 1e-4"
    return {"max_abs": float(diff.max()), "max_over_bound": float((diff / bound).max()),
            "exact": float((g == wnt).mean())}


@pytest.mark.parametrize("out,n_in,norm,res", [
    (6144, 2560, True, False),     # q/k/v of one Qwen3-4B layer, input RMSNorm fused
    (2560, 4096, False, True),     # o_proj + residual
    (2560, 9728, False, True),     # down_proj + residual
    (151936, 2560, True, False),   # lm_head with the final RMSNorm (4 rows per wave)
    (1001, 40, True, True),        # ragged: rows off the workgroup size, 5 chunks per row
    (1029, 2560, True, True),      # ten-wave workgroups with the fused RMSNorm, a partial last workgroup
    (16389, 8, False, False),      # 4-row path with a partial last wave, one chunk per row
    (37, 16384, True, False),      # the largest input
])
def test_gemv_matches_float64_reference(out, n_in, norm, res):
    from nova_amd.gemv import rms_gemv

    print(f"case gemv out={out} in={n_in} norm={norm} residual={res}", flush=True)
    x = _x(n_in, 1, 3.0)
    w = _w(out, n_in, 2)
    gamma = (1.0 + 0.2 * _x(n_in, 3)).half() if norm else None
    residual = _x(out, 4) if res else None
    got = rms_gemv(x, w, gamma, EPS, residual)
    torch.cuda.synchronize()
    want = _ref_gemv(x, w, gamma, residual)
    st = _check(got, want, x, w, gamma, residual, f"gemv {out}x{n_in}")
    print(f"  {st}", flush=True)


def test_gemv_in_place_residual_and_errors():
    from nova_amd.gemv import rms_gemv

    x, w, r = _x(9728, 5), _w(2560, 9728, 6), _x(2560, 7)
    want = _ref_gemv(x, w, None, r)
    h = r.clone()
    rms_gemv(x, w, residual=h, out=h)  # the decoder's down_proj: h += W act, in place
    _check(h, want, x, w, None, r, "in place")
    with pytest.raises(ValueError, match="alias"):
        rms_gemv(x[:2560], _w(2560, 2560, 1), out=x[:2560])
    with pytest.raises(ValueError, match="multiple of 8"):
        rms_gemv(_x(100, 1), _w(10, 100, 1))
    with pytest.raises(ValueError, match="16384"):
        rms_gemv(_x(16392, 1), _w(4, 16392, 1))
    with pytest.raises(ValueError, match="fp16"):
        rms_gemv(_x(64, 1).float(), _w(4, 64, 1))


@pytest.mark.parametrize("inter,n_in", [(9728, 2560), (999, 64)])
def test_swiglu_gemv_matches_float64_reference(inter, n_in):
    from nova_amd.gemv import swiglu_gemv

    print(f"case swiglu inter={inter} in={n_in}", flush=True)
    x = _x(n_in, 11, 2.0)
    wgu = _w(2 * inter, n_in, 12)
    gamma = (1.0 + 0.2 * _x(n_in, 13)).half()
    got = swiglu_gemv(x, wgu, gamma, EPS)
    torch.cuda.synchronize()
    gu = (wgu.double() @ _rms16(x, gamma).double()).half()
    g, u = gu[:inter], gu[inter:]
    want = F.silu(g) * u  # fp16 ops, as LeanMLP evaluates them
    st = assert_ulp_or_abs(npy(got), npy(want.float()), 3, 1e-4, f"swiglu {inter}x{n_in}")
    print(f"  {st}", flush=True)


@pytest.mark.parametrize("pos", [0, 1, 4095, 32767, 65600])
def test_qk_norm_rope_matches_skeleton_torch_ops(pos):
    from nova_amd.gemv import qk_norm_rope_
    from nova_amd.skeleton import _rms, _rotate_half

    hq, hkv, d = 32, 8, 128
    qkv = _x((hq + 2 * hkv) * d, 21, 4.0)
    qg, kg = (1.0 + 0.3 * _x(d, 22)).half(), (1.0 + 0.3 * _x(d, 23)).half()
    inv = 1.0 / (1_000_000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    inv = inv.cuda()
    p = torch.tensor([pos], dtype=torch.int64, device="cuda")
    # the skeleton's torch path for one token (SkeletonText._layers_torch + SkeletonAttention.forward)
    freqs = p.float()[..., None] * inv
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos().half(), emb.sin().half()
    q = _rms(qkv[:hq * d].view(hq, d), qg, EPS)
    k = _rms(qkv[hq * d:(hq + hkv) * d].view(hkv, d), kg, EPS)
    t1 = torch.cat([(t * cos).reshape(-1) for t in (q, k)])
    t2 = torch.cat([(_rotate_half(t) * sin).reshape(-1) for t in (q, k)])
    want = torch.cat([t1 + t2, qkv[(hq + hkv) * d:]])
    got = qk_norm_rope_(qkv.clone(), hq, hkv, qg, kg, EPS, inv, p)
    torch.cuda.synchronize()
    # the head norm's factor can sit a float ULP away from torch's (another summation order
    # over 128 elements), which flips the fp16 rounding of a normalized element now and then:
    # each element within one flip of each RoPE term plus one of the sum
    n = t1.numel()
    g, w = npy(got[:n]).astype(np.float64), npy(want[:n]).astype(np.float64)
    diff = np.abs(g - w)
    bound = _spacing16(npy(t1)) + _spacing16(npy(t2)) + _spacing16(w)
    assert int((diff > bound).sum()) == 0, f"pos={pos}: {int((diff > bound).sum())} elements beyond the bound"
    exact = float((g == w).mean())
    print(f"pos={pos} exact {exact:.4f} max abs {diff.max():.2e}", flush=True)
    assert torch.equal(got[n:], qkv[n:])  # v untouched
    assert exact > 0.98


def _decoder_pair(cfg, prompt: int, max_len: int = 512):
    from nova_amd.decode import GraphDecoder
    from nova_amd.skeleton import SkeletonForCausalLM

    model = SkeletonForCausalLM(cfg, seed=0).half().cuda().eval()
    ids = torch.randint(0, cfg.vocab_size, (1, prompt), generator=torch.Generator().manual_seed(9)).cuda()
    return model, ids, GraphDecoder


def test_kernel_decoder_tracks_torch_decoder_and_replays_bitwise():
    """A 4-layer decoder with the SwiGLU MLP: the kernel-mode decode steps stay close to the
    torch-mode steps from the same token (relative logit difference < 1e-2, the same greedy
    token nearly always), and kernel-mode graph replays equal eager kernel-mode steps bit for
    bit (every kernel on the path is deterministic)."""
    from nova_amd.skeleton import SkeletonConfig

    cfg = SkeletonConfig(num_hidden_layers=4, hidden_size=1024, intermediate_size=2816, vocab_size=4096)
    model, ids, GraphDecoder = _decoder_pair(cfg, 300)
    tdec = GraphDecoder(model, max_len=512, quant="int8")
    tdec.prefill(ids)
    tdec.capture(warmup=2)
    torch_logits, torch_ids = [], []
    start = tdec.input_ids.clone()
    for _ in range(6):
        torch_ids.append(tdec.input_ids.clone())
        tdec.step()
        torch_logits.append(tdec.logits.float().clone())

    model.use_decode_kernels(True)
    kdec, edec = GraphDecoder(model, max_len=512, quant="int8"), GraphDecoder(model, max_len=512, quant="int8")
    for dec in (kdec, edec):
        dec.prefill(ids)
        dec.input_ids.copy_(start)
    kdec.capture(warmup=2)
    rels, agree = [], 0
    for i in range(6):
        kdec.input_ids.copy_(torch_ids[i])
        edec.input_ids.copy_(torch_ids[i])
        kdec.step()
        with torch.inference_mode():
            eager = edec._body()
        torch.cuda.synchronize()
        assert torch.equal(kdec.logits, eager), f"step {i}: replay != eager"
        assert torch.equal(kdec.input_ids, edec.input_ids)
        a, b = kdec.logits.float(), torch_logits[i]
        rels.append(float((a - b).norm() / b.norm()))
        agree += int(torch.equal(a.argmax(-1), b.argmax(-1)))
    print(f"kernel vs torch relative logit differences {[f'{r:.1e}' for r in rels]}, argmax agree {agree}/6",
          flush=True)
    assert max(rels) < 1e-2, rels
    assert agree >= 5
    assert int(kdec.cache.pos.item()) == 300 + 6
    model.use_decode_kernels(False)
