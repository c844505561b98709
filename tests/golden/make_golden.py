"""Write golden vectors for the int8 KV path from the reference implementation itself.

Run in the build container only (it reads the reference sources from
``/root/reference/src``; nothing on the GPU side runs this script):

    python tests/golden/make_golden.py

What it records, and why a golden vector is needed for it:

- ``quant_*.npz``: ``nova.kvquant.quantize_int8`` / ``dequantize_int8`` outputs
  (``src/nova/kvquant.py:118-176``) on seeded inputs, including the
  replicate-pad lengths, channel outliers, constant groups, the 1e-8 step floor
  and large magnitudes. Closed-form invariants cannot tell whether codes are
  computed with the fp32 step or its fp16 rounding; these vectors can.
- ``stream.npz``: the state of ``nova.kvattn.KVInt8Cache`` (device="cpu")
  through a chunked prefill and 70 decode appends that cross a group
  boundaries (``src/nova/kvattn.py:636-833``): codes, rulers, ring, scalars
  and ring masks, plus ``tail_attend`` outputs (``kvattn.py:447-482``).
- ``bytes.json``: ``bytes_per_token`` int8 accounting (``kvquant.py:232-289``).

Inputs come from ``torch.Generator().manual_seed(...)`` on the CPU, so the
vectors are reproducible without a GPU.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

REF_SRC = Path("/root/reference/src")
OUT = Path(__file__).resolve().parent


def _ref():
    sys.path.insert(0, str(REF_SRC))
    import nova.kvattn as kvattn  # noqa: E402
    import nova.kvquant as kvquant  # noqa: E402
    return kvquant, kvattn


def _x(shape, seed: int, scale: float = 1.0, outlier_channels=(), outlier_gain: float = 8.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    for c in outlier_channels:
        x[..., c] *= outlier_gain
    return x.to(torch.float16)


def quant_cases(kvquant) -> None:
    cases = {}
    # token axis, group 64: lengths on and off the group boundary (replicate pad)
    for n, seed in ((37, 0), (64, 1), (130, 2), (200, 3)):
        cases[f"tok64_n{n}"] = (_x((1, 2, n, 128), seed, 1.0, (3, 71, 120), 8.0), 64, "token")
    # the bench's outlier construction: 4 seeded channels x8 per head, 8 heads
    x = _x((1, 8, 96, 128), 4)
    g = torch.Generator().manual_seed(5)
    for h in range(8):
        ch = torch.randperm(128, generator=g)[:4]
        x[0, h, :, ch] = (x[0, h, :, ch].float() * 8).to(torch.float16)
    cases["tok64_bench_outliers"] = (x, 64, "token")
    # whole-sequence group (group_size 0) and a small group
    cases["tok0_n50"] = (_x((1, 2, 50, 128), 6), 0, "token")
    cases["tok4_n10"] = (_x((1, 2, 10, 128), 7, 3.0), 4, "token")
    # degenerate rulers: constant tensor, tiny range (1e-8 floor), large magnitude, negative offset
    const = torch.full((1, 2, 64, 128), 3.5, dtype=torch.float16)
    tiny = (torch.full((1, 1, 64, 128), 0.25) + _x((1, 1, 64, 128), 8).float() * 1e-7).to(torch.float16)
    big = _x((1, 1, 64, 128), 9, 8000.0)  # |x| stays below the fp16 max
    offset = (_x((1, 1, 64, 128), 10, 0.05).float() + 100.0).to(torch.float16)
    sub = _x((1, 1, 64, 128), 11, 1e-6)  # fp16 subnormals
    cases["tok64_special"] = (torch.cat([const[:, :1], tiny, big, offset, sub], dim=1), 64, "token")
    # channel axis (the default axis of quantize_int8)
    cases["chan32_n37"] = (_x((1, 4, 37, 128), 12, 3.0), 32, "channel")
    cases["chan0_n9"] = (_x((1, 2, 9, 128), 13), 0, "channel")

    for name, (x, gs, axis) in cases.items():
        q, mn, st = kvquant.quantize_int8(x, gs, axis)
        dq = kvquant.dequantize_int8(q, mn, st, gs, axis)
        np.savez_compressed(OUT / f"quant_{name}.npz", x=x.numpy(), q=q.numpy(), mins=mn.numpy(),
                            steps=st.numpy(), deq=dq.numpy(), group=np.int64(gs),
                            axis=np.array(axis))


def stream_case(kvattn) -> None:
    """Chunked prefill of 130 tokens (chunks of 96), then 70 decode appends."""
    hkv, hq, d, max_len, n0, steps = 2, 8, 128, 320, 130, 70
    k = _x((1, hkv, n0 + steps, d), 20, 0.7)
    v = _x((1, hkv, n0 + steps, d), 21, 0.7)
    q = _x((1, hq, 1, d), 22, 0.7)
    cache = kvattn.KVInt8Cache(num_slots=1, num_kv_heads=hkv, head_dim=d, max_len=max_len,
                               num_q_heads=hq, device="cpu")
    cache.begin_prefill(n0)
    for c0 in range(0, n0, 96):
        nc = min(96, n0 - c0)
        cache.set_prefill_pos(c0)
        cache.update(k[:, :, c0:c0 + nc], v[:, :, c0:c0 + nc], 0)
    cache.finish_prefill(n0)
    rec = {"k": k.numpy(), "v": v.numpy(), "q": q.numpy(), "n0": np.int64(n0),
           "max_len": np.int64(max_len)}

    def snap(tag: str) -> None:
        rec[f"{tag}_kq"] = cache.kq[0].numpy().copy()
        rec[f"{tag}_vq"] = cache.vq[0].numpy().copy()
        for nm in ("kmn", "kst", "vmn", "vst"):
            rec[f"{tag}_{nm}"] = getattr(cache, nm)[0].numpy().copy()
        rec[f"{tag}_tail_k"] = cache.tail_k[0].numpy().copy()
        rec[f"{tag}_tail_v"] = cache.tail_v[0].numpy().copy()

    snap("prefill")
    rec["prefill_scalars"] = np.array([int(cache.pos), int(cache.first), int(cache._written),
                                       int(cache._qlen), int(cache._pg)], np.int64)
    scal, masks, touts, tlses = [], [], [], []
    for i in range(steps):
        p = n0 + i
        cache.pos.fill_(p)
        cache.update(k[:, :, p:p + 1], v[:, :, p:p + 1], 0)
        scal.append([int(cache._written), int(cache._qlen), int(cache._pg)])
        mask = cache.ring_mask()
        masks.append(mask.view(-1).numpy().copy())
        to, tl = kvattn.tail_attend(q, cache.tail_k[0], cache.tail_v[0], mask)
        touts.append(to.numpy().copy())
        tlses.append(tl.numpy().copy())
        if p in (191, 192, 199):
            snap(f"step{p}")
    rec["step_scalars"] = np.array(scal, np.int64)
    rec["step_masks"] = np.array(masks, bool)
    rec["tail_out"] = np.array(touts)
    rec["tail_lse"] = np.array(tlses)
    np.savez_compressed(OUT / "stream.npz", **rec)


def bytes_case(kvquant) -> None:
    out = {
        "c8": kvquant.bytes_per_token(36, 8, 128, bits=8),
        "c8t": kvquant.bytes_per_token(36, 8, 128, bits=8, k_axis="token", token_group=64),
    }
    (OUT / "bytes.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")


def main() -> None:
    kvquant, kvattn = _ref()
    quant_cases(kvquant)
    stream_case(kvattn)
    bytes_case(kvquant)
    for f in sorted(OUT.glob("*.npz")) + [OUT / "bytes.json"]:
        print(f"{f.name:40s} {f.stat().st_size:8d} B")


if __name__ == "__main__":
    main()
