"""The CPU oracle, pinned: golden vectors written by the reference, closed forms and library routines.

Each check is chosen so that a plausible slip in the oracle (codes from the fp16
step instead of the fp32 step, truncation instead of round-half-even, a dropped
replicate pad, a transposed GQA head map, a wrong ring-slot formula) fails here.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attn as oattn
from oracle import decode as odec
from oracle import kvquant as okq
from oracle import stream as ostream

GOLD = Path(__file__).resolve().parent / "golden"
QUANT_FILES = sorted(GOLD.glob("quant_*.npz"))


# ---------------------------------------------------------------- quantizer vs reference vectors


@pytest.mark.parametrize("path", QUANT_FILES, ids=[p.stem for p in QUANT_FILES])
def test_quantizer_matches_reference_vectors(path):
    z = np.load(path)
    gs, axis = int(z["group"]), str(z["axis"])
    q, mn, st = okq.quantize_int8(z["x"], gs, axis)
    assert q.dtype == np.uint8 and mn.dtype == np.float16 and st.dtype == np.float16
    np.testing.assert_array_equal(q, z["q"])
    np.testing.assert_array_equal(mn.view(np.uint16), z["mins"].view(np.uint16))
    np.testing.assert_array_equal(st.view(np.uint16), z["steps"].view(np.uint16))
    deq = okq.dequantize_int8(z["q"], z["mins"], z["steps"], gs, axis)
    np.testing.assert_array_equal(deq.view(np.uint16), z["deq"].view(np.uint16))


def test_vectors_pin_fp32_step_for_codes():
    """A quantizer that divided by the stored fp16 step would still pass every invariant;
    the reference vectors must reject it."""
    diffs = 0
    for path in QUANT_FILES:
        z = np.load(path)
        if str(z["axis"]) != "token" or int(z["group"]) != 64:
            continue
        x = z["x"].astype(np.float32)
        *lead, n, dim = x.shape
        pad = (-n) % 64
        xp = np.take(x, np.minimum(np.arange(n + pad), n - 1), axis=-2)
        g = xp.reshape(*lead, (n + pad) // 64, 64, dim)
        mn = g.min(axis=-2)
        st16 = z["steps"].astype(np.float32)
        wrong = np.clip(np.rint((g - mn[..., None, :]) / np.maximum(st16, 1e-8)[..., None, :]), 0, 255)
        wrong = wrong.astype(np.uint8).reshape(*lead, n + pad, dim)[..., :n, :]
        diffs += int((wrong != z["q"]).sum())
    assert diffs > 0


def test_vectors_pin_round_half_even():
    """Truncation (or round-half-away) instead of rint must disagree with the vectors."""
    z = np.load(GOLD / "quant_tok64_n200.npz")
    x = z["x"].astype(np.float32)
    *lead, n, dim = x.shape
    xp = np.take(x, np.minimum(np.arange(n + 56), n - 1), axis=-2).reshape(*lead, 4, 64, dim)
    mn = xp.min(axis=-2)
    step = np.maximum((xp.max(axis=-2) - mn) / np.float32(255), np.float32(1e-8))
    r = (xp - mn[..., None, :]) / step[..., None, :]
    trunc = np.clip(np.floor(r), 0, 255).astype(np.uint8).reshape(*lead, 256, dim)[..., :n, :]
    assert (trunc != z["q"]).any()


# ---------------------------------------------------------------- quantizer closed forms


def test_constant_tensor_round_trips_exactly():
    """``max == min``: step floors at 1e-8, codes are 0, the round trip is lossless
    (``tests/test_kvquant.py:243-249``)."""
    const = np.full((1, 2, 8, 128), 3.5, np.float16)
    for axis, gs in (("channel", 32), ("token", 4)):
        q, mn, st = okq.quantize_int8(const, gs, axis)
        assert q.shape == const.shape
        assert not q.any()
        np.testing.assert_array_equal(okq.dequantize_int8(q, mn, st, gs, axis), const)


@pytest.mark.parametrize("n", [1, 37, 63, 64, 65, 130])
def test_token_axis_invariants(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((2, 3, n, 128)) * 2.0).astype(np.float16)
    q, mn, st = okq.quantize_int8_token(x, 64)
    ng = -(-n // 64)
    assert q.shape == x.shape and mn.shape == st.shape == (2, 3, ng, 128)
    xf = x.astype(np.float32)
    pad = np.take(xf, np.minimum(np.arange(ng * 64), n - 1), axis=-2).reshape(2, 3, ng, 64, 128)
    # the ruler is the group's true min (exact in fp16) and its span / 255
    np.testing.assert_array_equal(mn.astype(np.float32), pad.min(axis=-2))
    span = pad.max(axis=-2) - pad.min(axis=-2)
    # min element codes to 0 and max element to 255 in every non-degenerate group
    qg = np.take(q, np.minimum(np.arange(ng * 64), n - 1), axis=-2).reshape(2, 3, ng, 64, 128)
    assert (qg.min(axis=-2) == 0).all()
    assert (qg.max(axis=-2)[span > 1e-3] == 255).all()
    # round trip within half a step, plus the drift of the fp16-stored step over up to
    # 255 codes (255 * 2^-11 of a step), plus the fp16 rounding of the result
    deq = okq.dequantize_int8_token(q, mn, st, 64).astype(np.float32)
    step16 = np.repeat(st.astype(np.float32), 64, axis=-2)[..., :n, :]
    err = np.abs(deq - xf)
    bound = step16 * (0.5 + 255 * 2.0 ** -11) * 1.01 + np.abs(xf) * 2.0 ** -11 + 1e-7
    assert (err <= bound).all()


def test_replicate_pad_equals_explicit_padding():
    """Padding by repeating the last token leaves min/max unchanged: quantizing n tokens
    equals quantizing the explicitly padded tensor and slicing."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 2, 37, 128)).astype(np.float16)
    xp = np.concatenate([x, np.repeat(x[:, :, -1:], 27, axis=2)], axis=2)
    a = okq.quantize_int8_token(x, 64)
    b = okq.quantize_int8_token(xp, 64)
    np.testing.assert_array_equal(a[0], b[0][:, :, :37])
    np.testing.assert_array_equal(a[1], b[1])
    np.testing.assert_array_equal(a[2], b[2])


def test_tok_scheme_closed_form():
    """Per-token symmetric scheme (extension): the absmax element codes to +-127 and the
    round trip stays within half a scale plus fp16 rounding."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((2, 50, 128)) * 3.0).astype(np.float16)
    q, s = okq.quantize_tok(x)
    assert q.dtype == np.int8 and s.shape == (2, 50)
    xf = x.astype(np.float32)
    am = np.abs(xf).argmax(axis=-1)
    top = np.take_along_axis(q, am[..., None], axis=-1)[..., 0]
    assert (np.abs(top.astype(np.int32)) == 127).all()
    assert (q >= -127).all()
    deq = okq.dequantize_tok(q, s).astype(np.float32)
    bound = s.astype(np.float32)[..., None] * 0.5 * 1.01 + np.abs(xf) * 2.0 ** -10 + 1e-7
    assert (np.abs(deq - xf) <= bound).all()
    z = np.zeros((1, 3, 128), np.float16)
    qz, sz = okq.quantize_tok(z)
    np.testing.assert_array_equal(okq.dequantize_tok(qz, sz), z)


def _tok_special_rows() -> np.ndarray:
    """Two fp16 rows of 128 whose codes pin the per-token symmetric quantizer's rounding:
    row 0 has absmax 127, so its fp32 scale is exactly 1.0 and x / scale is x itself: the ties
    +-0.5, +-1.5, +-2.5, 3.5 code to 0, 0, +-2, +-2, 4 under round-half-to-even (half away from
    zero would give +-1, +-2, +-3, 4). Row 1 has absmax 3: fp32 scale 3 / 127, fp16 scale
    0.02362060546875 (0x260C); 1.759765625 / fp32 scale = 74.4967.. codes to 74, while dividing
    by the fp16 scale (74.502..) would give 75."""
    x = np.zeros((2, 128), np.float16)
    x[0, :8] = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5]
    x[1, :3] = [3.0, 1.759765625, -1.759765625]
    return x


TOK_SPECIAL_CODES = ([127, 0, 0, 2, -2, 2, -2, 4], [127, 74, -74])
TOK_SPECIAL_SCALES = (0x3C00, 0x260C)


def test_tok_scheme_rounding_conventions():
    """The tie and scale-rounding rows code to the literal values above, and both pins
    discriminate: half-away-from-zero rounding, or codes computed with the stored fp16 scale,
    would differ on them."""
    from fractions import Fraction

    x = _tok_special_rows()
    q, s = okq.quantize_tok(x)
    for r in range(2):
        want = np.zeros(128, np.int8)
        want[:len(TOK_SPECIAL_CODES[r])] = TOK_SPECIAL_CODES[r]
        np.testing.assert_array_equal(q[r], want)
        assert int(s[r:r + 1].view(np.uint16)[0]) == TOK_SPECIAL_SCALES[r]
    # the alternatives the rows rule out
    half_away = np.sign(x[0, :8].astype(np.float32)) * np.floor(np.abs(x[0, :8].astype(np.float32)) + 0.5)
    assert not np.array_equal(half_away.astype(np.int8), q[0, :8])
    by_fp16_scale = np.rint(np.float32(1.759765625) / s[1].astype(np.float32))
    assert by_fp16_scale == 75 and q[1, 1] == 74
    # 74: the exact quotient by the fp32 scale, in rationals
    s32 = np.float32(np.float32(3.0) / np.float32(127.0))
    assert round(Fraction(1.759765625) / Fraction(float(s32))) == 74


def test_bytes_accounting_matches_reference():
    """``tests/test_kvquant.py:261-270``: int8 is 1.85-1.95x smaller and ~77.6 KiB/token."""
    gold = json.loads((GOLD / "bytes.json").read_text())
    c8 = okq.bytes_per_token_int8(36, 8, 128)
    c8t = okq.bytes_per_token_int8(36, 8, 128, k_axis="token", token_group=64)
    assert c8 == pytest.approx(gold["c8"])
    assert c8t == pytest.approx(gold["c8t"])
    assert 1.85 <= c8["ratio"] <= 1.95 and 1.85 <= c8t["ratio"] <= 1.95
    assert abs(c8["int8_kv"] / 1024 - 77.6) < 1.0


# ---------------------------------------------------------------- attention oracle


def _rand(shape, seed, scale=0.7):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float16)


def test_attention_matches_torch_math_sdpa():
    """The fp64 oracle agrees with torch's math SDPA (fp32 upcast) on repeat-kv expanded K/V."""
    hq, hkv, n, d = 8, 2, 150, 128
    q, k, v = _rand((hq, d), 0), _rand((hkv, n, d), 1), _rand((hkv, n, d), 2)
    out, _ = oattn.attend_fp16_kv(q, k, v)
    kt = torch.from_numpy(k).float().repeat_interleave(hq // hkv, 0)[None]
    vt = torch.from_numpy(v).float().repeat_interleave(hq // hkv, 0)[None]
    qt = torch.from_numpy(q).float()[None, :, None]
    want = F.scaled_dot_product_attention(qt, kt, vt, scale=d ** -0.5)[0, :, 0].double().numpy()
    np.testing.assert_allclose(out, want, rtol=0, atol=2e-6)


def test_attention_special_cases():
    d = 128
    q = _rand((8, d), 3)
    # one token: the output is that token's V for every head of the group
    k1, v1 = _rand((2, 1, d), 4), _rand((2, 1, d), 5)
    out, lse = oattn.attend_fp16_kv(q, k1, v1)
    np.testing.assert_allclose(out[:4], np.repeat(v1[0].astype(np.float64), 4, 0))
    np.testing.assert_allclose(out[4:], np.repeat(v1[1].astype(np.float64), 4, 0))
    np.testing.assert_allclose(lse[:4], (q[:4].astype(np.float64) @ k1[0, 0].astype(np.float64)) * d ** -0.5)
    # constant V per KV head: Q head h returns KV head h // 4's constant (test_kvattn.py:130-139)
    k = _rand((2, 40, d), 6)
    v = np.broadcast_to(np.arange(2, dtype=np.float16)[:, None, None], (2, 40, d))
    out, _ = oattn.attend_fp16_kv(q, k, v)
    np.testing.assert_allclose(out[:, 0], np.arange(8) // 4, atol=1e-12)
    # identical keys: uniform weights, the output is the mean of V
    kk = np.broadcast_to(_rand((2, 1, d), 7), (2, 5, d))
    vv = _rand((2, 5, d), 8)
    out, _ = oattn.attend_fp16_kv(q, kk, vv)
    np.testing.assert_allclose(out[:4], np.repeat(vv[0].astype(np.float64).mean(0, keepdims=True), 4, 0))


def test_int8_decode_oracle_used_zero_and_garbage():
    hq, hkv, d = 8, 2, 128
    q = _rand((hq, d), 9)
    k, v = _rand((hkv, 300, d), 10), _rand((hkv, 300, d), 11)
    kq, kmn, kst = okq.quantize_int8_token(k, 64)
    vq, vmn, vst = okq.quantize_int8_token(v, 64)
    out0, lse0 = oattn.int8_attn_decode(q, kq, kmn, kst, vq, vmn, vst, 0)
    assert not out0.any() and np.isneginf(lse0).all()
    a, _ = oattn.int8_attn_decode(q, kq, kmn, kst, vq, vmn, vst, 250)
    kq2 = kq.copy()
    kq2[:, 250:] = 255
    b, _ = oattn.int8_attn_decode(q, kq2, kmn, kst, vq, vmn, vst, 250)
    np.testing.assert_array_equal(a, b)


def test_lse_merge_equals_single_softmax():
    """Merging two disjoint partials by log-sum-exp equals one softmax over the union."""
    hq, d = 8, 128
    q = _rand((hq, d), 12)
    k, v = _rand((2, 90, d), 13), _rand((2, 90, d), 14)
    o1, l1 = oattn.attend_fp16_kv(q, k[:, :60], v[:, :60])
    o2, l2 = oattn.attend_fp16_kv(q, k[:, 60:], v[:, 60:])
    whole, _ = oattn.attend_fp16_kv(q, k, v)
    merged = oattn.lse_merge(o1, l1, o2, l2)
    np.testing.assert_array_equal(merged, whole.astype(np.float16))
    # an empty side has lse -inf and weight 0
    e = oattn.lse_merge(o1, l1, np.zeros_like(o1), np.full(hq, -np.inf))
    np.testing.assert_array_equal(e, o1.astype(np.float16))


# ---------------------------------------------------------------- streaming cache vs reference vectors


def _replay_stream():
    z = np.load(GOLD / "stream.npz")
    k, v, q = z["k"][0], z["v"][0], z["q"][0, :, 0]
    n0, max_len = int(z["n0"]), int(z["max_len"])
    c = ostream.StreamCache(1, k.shape[0], k.shape[2], max_len, q.shape[0])
    c.begin_prefill(n0)
    for c0 in range(0, n0, 96):
        nc = min(96, n0 - c0)
        c.set_prefill_pos(c0)
        c.update(k[:, c0:c0 + nc], v[:, c0:c0 + nc], 0)
    c.finish_prefill(n0)
    return z, c, k, v, q, n0


def _assert_state(z, c, tag):
    np.testing.assert_array_equal(c.kq[0], z[f"{tag}_kq"][0])
    np.testing.assert_array_equal(c.vq[0], z[f"{tag}_vq"][0])
    for nm in ("kmn", "kst", "vmn", "vst", "tail_k", "tail_v"):
        np.testing.assert_array_equal(getattr(c, nm)[0].view(np.uint16), z[f"{tag}_{nm}"][0].view(np.uint16))


def test_stream_state_matches_reference_vectors():
    z, c, k, v, q, n0 = _replay_stream()
    _assert_state(z, c, "prefill")
    assert [c.pos, c.first, c.written, c.qlen, c.pg] == list(z["prefill_scalars"])
    for i in range(z["step_scalars"].shape[0]):
        p = n0 + i
        c.pos = p
        c.update(k[:, p:p + 1], v[:, p:p + 1], 0)
        assert [c.written, c.qlen, c.pg] == list(z["step_scalars"][i]), p
        mask = c.ring_mask()
        np.testing.assert_array_equal(mask, z["step_masks"][i])
        assert mask.sum() == c.written - c.qlen
        to, tl = oattn.tail_attend(q, c.tail_k[0], c.tail_v[0], mask)
        ref_o = z["tail_out"][i][0, :, 0]
        ref_l = z["tail_lse"][i][0]
        np.testing.assert_allclose(to.astype(np.float32), ref_o.astype(np.float32), atol=2e-3, rtol=0)
        np.testing.assert_allclose(tl, ref_l, rtol=1e-5, atol=1e-5)
        if f"step{p}_kq" in z:
            _assert_state(z, c, f"step{p}")


def test_full_ring_requant_equals_quantizer():
    """When slot 63 of a group is written, the requantized ring equals ``quantize_int8``
    of that aligned 64-token group."""
    z, c, k, v, q, n0 = _replay_stream()
    for p in range(n0, 192):
        c.pos = p
        c.update(k[:, p:p + 1], v[:, p:p + 1], 0)
    kq, kmn, kst = okq.quantize_int8_token(k[:, 128:192], 64)
    np.testing.assert_array_equal(c.kq[0][:, 128:192], kq)
    np.testing.assert_array_equal(c.kmn[0][:, 2], kmn[:, 0])
    np.testing.assert_array_equal(c.kst[0][:, 2], kst[:, 0])
    assert c.qlen == 192 and not c.ring_mask().any()


def test_stream_two_part_equals_exact_within_streaming_tolerance():
    z, c, k, v, q, n0 = _replay_stream()
    for p in range(n0, n0 + 20):
        c.pos = p
        c.update(k[:, p:p + 1], v[:, p:p + 1], 0)
    a = c.attend_two_part(q, 0).astype(np.float32)
    b = c.attend_exact(q, 0).astype(np.float32)
    assert np.abs(a - b).max() <= 1e-3


# ---------------------------------------------------------------- decoder buckets


def test_bucket_for_table():
    """``tests/test_decode_mask_bucket.py:29-37``."""
    assert odec.bucket_for(1) == 2070
    assert odec.bucket_for(2070) == 2070
    assert odec.bucket_for(2071) == 4096
    assert odec.bucket_for(8192) == 8192
    assert odec.bucket_for(16384 + 64) == 32768
    assert odec.bucket_for(65536) == 65536
    assert odec.bucket_for(70000) == 70000


def test_mask_row_matches_table():
    """Row ``pos`` of the lower-triangular additive table (``decode.py:176-189``)."""
    max_len = 64
    neg = np.finfo(np.float16).min
    idx = np.arange(max_len)
    table = np.where(idx[None, :] <= idx[:, None], np.float16(0), np.float16(neg))
    for pos in (0, 1, 7, 63):
        np.testing.assert_array_equal(odec.mask_row(pos, max_len), table[pos])


def test_chunk_prefill_oracle_pinned():
    """The chunked-prefill oracle against independent routes: the last query token sees
    every key (== ``attend_fp16_kv`` over the whole dequantized cache + chunk), the first
    sees only the cache and itself, torch's math SDPA with an explicit causal mask agrees
    on every row, and a constant V comes back (to fp64 rounding)."""
    import torch

    rng = np.random.default_rng(7)
    hkv, gq, d, used, m = 2, 4, 128, 128, 40
    hq = hkv * gq
    kc = (rng.standard_normal((hkv, used, d)) * 0.7).astype(np.float16)
    vc = (rng.standard_normal((hkv, used, d)) * 0.7).astype(np.float16)
    kq, kmn, kst = okq.quantize_int8_token(kc, 64)
    vq, vmn, vst = okq.quantize_int8_token(vc, 64)
    k_ch = (rng.standard_normal((hkv, m, d)) * 0.7).astype(np.float16)
    v_ch = (rng.standard_normal((hkv, m, d)) * 0.7).astype(np.float16)
    q = (rng.standard_normal((hq, m, d)) * 0.7).astype(np.float16)
    got = oattn.chunk_prefill_attend(q, kq, kmn, kst, vq, vmn, vst, used, k_ch, v_ch)
    k16 = okq.dequantize_int8_token(kq, kmn, kst, 64)
    v16 = okq.dequantize_int8_token(vq, vmn, vst, 64)
    kall = np.concatenate([k16, k_ch], 1)
    vall = np.concatenate([v16, v_ch], 1)
    last, _ = oattn.attend_fp16_kv(q[:, m - 1], kall, vall)
    np.testing.assert_allclose(got[:, m - 1], last, rtol=0, atol=1e-12)
    first, _ = oattn.attend_fp16_kv(q[:, 0], kall[:, :used + 1], vall[:, :used + 1])
    np.testing.assert_allclose(got[:, 0], first, rtol=0, atol=1e-12)
    qt = torch.from_numpy(q.astype(np.float64))
    kt = torch.from_numpy(kall.astype(np.float64)).repeat_interleave(gq, 0)
    vt = torch.from_numpy(vall.astype(np.float64)).repeat_interleave(gq, 0)
    mask = torch.arange(used + m)[None, :] <= (used + torch.arange(m))[:, None]
    sd = torch.nn.functional.scaled_dot_product_attention(qt[None], kt[None], vt[None], attn_mask=mask)[0]
    np.testing.assert_allclose(got, sd.numpy(), rtol=0, atol=1e-10)
    vconst = np.full_like(v_ch, 0.375)
    vqc, vmc, vsc = okq.quantize_int8_token(np.full_like(vc, 0.375), 64)
    const = oattn.chunk_prefill_attend(q, kq, kmn, kst, vqc, vmc, vsc, used, k_ch, vconst)
    np.testing.assert_allclose(const, np.full_like(const, 0.375), rtol=0, atol=1e-12)


@pytest.mark.parametrize("used,hist", [(0, 192), (512, 192), (128, 5)])
def test_chunk_prefill_with_fp16_history(used, hist):
    """An fp16 history before the chunk (the staged prefill's later chunks): against torch's
    SDPA in float64 with the causal mask shifted by the history, and equal to the last rows of
    the same attention computed for history and chunk together as one chunk (the rows of a
    causal attention do not depend on the other queries)."""
    rng = np.random.default_rng(used + hist)
    hq, hkv, d, n = 8, 2, 128, 37
    m = hist + n
    kc = (rng.standard_normal((hkv, max(used, 64), d)) * 0.7).astype(np.float16)
    vc = (rng.standard_normal((hkv, max(used, 64), d)) * 0.7).astype(np.float16)
    kq, kmn, kst = okq.quantize_int8_token(kc, 64)
    vq, vmn, vst = okq.quantize_int8_token(vc, 64)
    k16 = (rng.standard_normal((hkv, m, d)) * 0.7).astype(np.float16)
    v16 = (rng.standard_normal((hkv, m, d)) * 0.7).astype(np.float16)
    q_all = (rng.standard_normal((hq, m, d)) * 0.7).astype(np.float16)
    q = q_all[:, hist:]
    got = oattn.chunk_prefill_attend(q, kq, kmn, kst, vq, vmn, vst, used, k16, v16)
    whole = oattn.chunk_prefill_attend(q_all, kq, kmn, kst, vq, vmn, vst, used, k16, v16)
    np.testing.assert_allclose(got, whole[:, hist:], rtol=0, atol=1e-13)
    kd = okq.dequantize_int8_token(kq, kmn, kst, 64)[:, :used]
    vd = okq.dequantize_int8_token(vq, vmn, vst, 64)[:, :used]
    kall = np.concatenate([kd, k16], 1).astype(np.float64)
    vall = np.concatenate([vd, v16], 1).astype(np.float64)
    kt = torch.from_numpy(kall).repeat_interleave(hq // hkv, 0)
    vt = torch.from_numpy(vall).repeat_interleave(hq // hkv, 0)
    mask = torch.arange(used + m)[None, :] <= (used + hist + torch.arange(n))[:, None]
    sd = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q.astype(np.float64))[None], kt[None],
                                                          vt[None], attn_mask=mask)[0]
    np.testing.assert_allclose(got, sd.numpy(), rtol=0, atol=1e-10)
    # the first query sees the whole history: dropping the history's last token changes it
    drop = lambda x: np.concatenate([x[:, :hist - 1], x[:, hist:hist + 1]], 1)  # noqa: E731
    short = oattn.chunk_prefill_attend(q[:, :1], kq, kmn, kst, vq, vmn, vst, used, drop(k16), drop(v16))
    assert np.abs(short[:, 0] - got[:, 0]).max() > 1e-6


# ---------------------------------------------------------------- torch fp32 restatement (CPU baseline)


@pytest.mark.parametrize("path", [p for p in QUANT_FILES if "tok64" in p.stem], ids=lambda p: p.stem)
def test_torch_dequant_matches_reference_vectors(path):
    """The CPU baseline's torch dequantization reproduces the reference's dequantized values
    bit for bit (vectors written by the reference, replicate pad included)."""
    from oracle import torch_ref

    z = np.load(path)
    got = torch_ref.dequantize_int8_token(torch.from_numpy(z["q"]), torch.from_numpy(z["mins"]),
                                          torch.from_numpy(z["steps"]), 64)
    np.testing.assert_array_equal(got.numpy().view(np.uint16), z["deq"].view(np.uint16))


def test_torch_decode_step_matches_oracle_stream():
    """The torch decode step (dequantized prefix + valid ring slots, GQA, fp32 softmax) equals
    the numpy oracle's exact single softmax within one fp16 rounding, at a ring that straddles
    a group boundary and with a nonzero ``first``."""
    from oracle import torch_ref

    rng = np.random.default_rng(11)
    hq, hkv, d, n0 = 8, 2, 128, 150
    sc = ostream.StreamCache(1, hkv, d, 256, hq)
    k = (rng.standard_normal((hkv, n0 + 3, d)) * 0.7).astype(np.float16)
    v = (rng.standard_normal((hkv, n0 + 3, d)) * 0.7).astype(np.float16)
    sc.begin_prefill(n0)
    sc.set_prefill_pos(0)
    sc.update(k[:, :n0], v[:, :n0], 0)
    sc.finish_prefill(n0)
    for t in range(3):
        sc.update(k[:, n0 + t:n0 + t + 1], v[:, n0 + t:n0 + t + 1], 0)
        sc.pos += 1
    q = (rng.standard_normal((hq, d)) * 0.7).astype(np.float16)
    for first in (0, sc.written - 10):
        sc.first = first
        want = sc.attend_exact(q, 0).astype(np.float64)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
        got = torch_ref.decode_step_t64(t(q), t(sc.kq[0]), t(sc.kmn[0]), t(sc.kst[0]), t(sc.vq[0]), t(sc.vmn[0]),
                                        t(sc.vst[0]), t(sc.tail_k[0]), t(sc.tail_v[0]), sc.written, first)
        got = got.numpy().astype(np.float64)
        spacing = np.abs(np.spacing(want.astype(np.float16)).astype(np.float64))
        assert np.all(np.abs(got - want) <= 1.01 * spacing + 1e-7), float(np.abs(got - want).max())
    # the ring mask agrees with the oracle's
    assert np.array_equal(torch_ref.ring_mask(sc.written, sc.qlen, sc.first).numpy(), sc.ring_mask())


def test_torch_tok_step_matches_oracle():
    from oracle import torch_ref

    rng = np.random.default_rng(12)
    hq, hkv, d, n = 8, 2, 128, 77
    x = (rng.standard_normal((hkv, n, d)) * 0.9).astype(np.float16)
    y = (rng.standard_normal((hkv, n, d)) * 0.9).astype(np.float16)
    kq, ks = okq.quantize_tok(x)
    vq, vs = okq.quantize_tok(y)
    q = (rng.standard_normal((hq, d)) * 0.7).astype(np.float16)
    want, _ = oattn.tok_attn_decode(q, kq, ks, vq, vs, n)
    t = torch.from_numpy
    got = torch_ref.decode_step_tok(t(q), t(kq), t(ks), t(vq), t(vs), n).numpy()
    spacing = np.abs(np.spacing(want.astype(np.float16)).astype(np.float64))
    assert np.all(np.abs(got.astype(np.float64) - want.astype(np.float64)) <= 1.01 * spacing + 1e-7)


def test_decode_trajectory_equals_step_by_step_state_machine():
    """The batched trajectory oracle equals the state machine's per-step single softmax (fp64 over
    the dequantized int8 prefix and the valid ring slots) at every step, across several group
    completions, from a prefill that ends inside a group."""
    rng = np.random.default_rng(21)
    hq, hkv, d, n0, S = 8, 2, 128, 100, 150
    k = (rng.standard_normal((hkv, n0 + S, d)) * 0.8).astype(np.float16)
    v = (rng.standard_normal((hkv, n0 + S, d)) * 0.8).astype(np.float16)
    qs = (rng.standard_normal((S, hq, d)) * 0.6).astype(np.float16)
    traj = ostream.decode_trajectory(k, v, qs, n0)
    sc = ostream.StreamCache(1, hkv, d, 256, hq)
    sc.begin_prefill(n0)
    sc.set_prefill_pos(0)
    sc.update(k[:, :n0], v[:, :n0], 0)
    sc.finish_prefill(n0)
    for i in range(S):
        p = n0 + i
        sc.pos = p
        sc.update(k[:, p:p + 1], v[:, p:p + 1], 0)
        n_g, qlen = sc.pg, sc.qlen
        k16 = okq.dequantize_int8_token(sc.kq[0][:, :qlen], sc.kmn[0][:, :n_g], sc.kst[0][:, :n_g], 64)
        v16 = okq.dequantize_int8_token(sc.vq[0][:, :qlen], sc.vmn[0][:, :n_g], sc.vst[0][:, :n_g], 64)
        m = sc.ring_mask()
        want, _ = oattn.attend_fp16_kv(qs[i], np.concatenate([k16, sc.tail_k[0][:, m]], 1),
                                       np.concatenate([v16, sc.tail_v[0][:, m]], 1))
        np.testing.assert_allclose(traj[i], want, rtol=1e-12, atol=1e-12, err_msg=f"step {i}")
