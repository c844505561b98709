"""Benchmark: int8-KV decode attention over 36 layers at 32k context on one MI355X.

Workload (the long-context decode configuration): 36 layers x (32 q heads, 8 KV heads,
head_dim 128), batch 1, int8t64 KV cache prefilled to 32768 tokens from seeded N(0,1)
fp16 K/V with 4 random K channels per head scaled x8. One decode step = for each layer
one fused append + attention launch (``KVInt8Cache.update_attend``) with that layer's
synthetic q/k/v, then ``pos += 1``; the step is captured once as a hipGraph and
replayed (one replay per token). W untimed replays, then K timed replays bracketed by
``torch.cuda.synchronize()`` and HIP events on the replay stream.

Each layer's step is two launches: the prefix kernel (the append and the split-K
partials over the int8 prefix) and the tail kernel (ring attention and the combine).

Prints one JSON line (the driver's contract). ``value`` = decode tokens/s of the whole
job. ``roofline`` refers to the dominant kernel, the prefix kernel: its algorithmic bytes
per launch / its average launch duration, timed with HIP events over K replays of a
graph holding only its 36 launches per step (``nkv_decode_step_partials_t64``, the same
kernel and arguments as in the full step); the tail kernel is timed the same way and
reported beside it. ``traffic`` comes from the committed rocprofv3 --pmc summary
(FETCH_SIZE + WRITE_SIZE per dispatch of the prefix kernel, scaled by what the same
counters read for the library's plain copy kernel of known size). ``cpu_baseline`` times
the numpy oracle (dequantize + softmax attention, threads over KV heads) on one layer for
~10-30 s and scales to the 36-layer step.

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--no-cpu-baseline] [--scheme t64|tok]

``--scheme tok`` runs the same workload on the per-token symmetric int8 format
(``KVInt8TokCache``: every token int8 with one fp16 scale per token and KV head).
    python bench.py --traffic-from FETCH_DIR WRITE_DIR   # summarize two rocprofv3 --pmc runs
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

LAYERS, HQ, HKV, D, CTX = 36, 32, 8, 128, 32768
HBM_PEAK_GBS = 8000.0
# the fused step's append per layer: K and V ring read (64 x 128 fp16 each per KV head),
# new token read and written into the ring, 64 code rows and 4 ruler rows written
APPEND_BYTES = 64 * 128 * 2 * 2 * HKV + 2 * 2 * 128 * 2 * HKV + 64 * 128 * 2 * HKV + 4 * 128 * 2 * HKV
Q_BYTES = HQ * D * 2
PREFIX_KERNEL = "attn_prefix_kernel"
COPY_KERNEL = "copy16_kernel"
TRAFFIC_FILE = ROOT / "profiles" / "attn_prefix_kernel_32k_traffic.txt"
TRAFFIC_FILE_TOK = ROOT / "profiles" / "attn_prefix_kernel_tok_32k_traffic.txt"
# per-token symmetric format: the new token read, its codes and scale written (8 KV heads)
APPEND_BYTES_TOK = 2 * 128 * 2 * HKV + 2 * 128 * HKV + 2 * 2 * HKV


def attn_bytes(u: int) -> int:
    """Algorithmic bytes of one layer's decode attention with ``u`` tokens written:
    int8 codes + fp16 rulers of whole groups (2176 B per token over 8 KV heads), fp16
    ring tokens (4096 B), q and out (16384 B)."""
    q = u // 64 * 64
    return 2176 * q + 4096 * (u - q) + 16384


def attn_bytes_tok(u: int) -> int:
    """Algorithmic bytes of one layer's decode attention over ``u`` tokens of the per-token
    symmetric format: int8 codes + one fp16 scale per token, K and V, 8 KV heads (2080 B
    per token), q and out (16384 B)."""
    return 2080 * u + 16384


def prefix_launch_bytes_tok(u: int) -> int:
    """One prefix-kernel launch of the per-token symmetric step: the ``u - 1`` tokens before
    the new one, q, and the append."""
    return 2080 * max(u - 1, 0) + Q_BYTES + APPEND_BYTES_TOK


def prefix_launch_bytes(u: int) -> int:
    """Algorithmic bytes of one prefix-kernel launch with ``u`` tokens written: int8 codes
    + fp16 rulers of the whole groups before the ring's group (2176 B per token over 8 KV
    heads), q, and the append."""
    prefix = max(u - 1, 0) // 64 * 64
    return 2176 * prefix + Q_BYTES + APPEND_BYTES


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--ctx", type=int, default=CTX)
    ap.add_argument("--parts", type=int, default=0, help="work units per KV head (0 = library default)")
    ap.add_argument("--splits", type=int, default=0, help="prefill: cache splits (0 = library default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--chunk", type=int, default=2048, help="e2e: streamed prefill chunk (a multiple of 64)")
    ap.add_argument("--workload", choices=("decode", "paged", "prefill", "e2e"), default="decode",
                    help="decode: one 32k sequence (the headline); paged: 8 ragged sequences in a paged cache; "
                         "prefill: a 512-token chunk over a 16384-token int8 cache (MFMA)")
    ap.add_argument("--scheme", choices=("t64", "tok"), default="t64",
                    help="KV format: int8t64 (the reference's) or per-token symmetric")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarize two rocprofv3 --pmc runs of this script into the traffic file")
    return ap.parse_args()


def _pmc_means(run_dir: str, counter: str) -> dict:
    """Mean per-dispatch value of ``counter`` for each kernel in a rocprofv3 --pmc CSV run."""
    import csv

    files = sorted(Path(run_dir).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {run_dir}")
    acc: dict = {}
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                name = row["Kernel_Name"]
                for key in (PREFIX_KERNEL, "attn_tail_kernel", COPY_KERNEL):
                    if key in name:
                        acc.setdefault(key, []).append(float(row["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def write_traffic(fetch_dir: str, write_dir: str, scheme: str = "t64") -> None:
    """Traffic of the prefix kernel from FETCH_SIZE and WRITE_SIZE (KiB per dispatch),
    each scaled by the factor that makes the same counter read the copy kernel's known
    byte count (COPY_BYTES read and written)."""
    fetch, write = _pmc_means(fetch_dir, "FETCH_SIZE"), _pmc_means(write_dir, "WRITE_SIZE")
    f_scale = COPY_BYTES / (fetch[COPY_KERNEL] * 1024)
    w_scale = COPY_BYTES / (write[COPY_KERNEL] * 1024)
    f_bytes = fetch[PREFIX_KERNEL] * 1024 * f_scale
    w_bytes = write[PREFIX_KERNEL] * 1024 * w_scale
    tok = scheme == "tok"
    alg = prefix_launch_bytes_tok(CTX + 1) if tok else prefix_launch_bytes(CTX + 1)
    flag = " --scheme tok" if tok else ""
    lines = [
        f"# HBM traffic of nkv::attn_prefix_kernel ({'per-token symmetric' if tok else 'int8t64'} format), "
        "32k-context decode step (36 layers, 32 q / 8 kv heads)",
        "# made by (rocprofv3 --pmc runs of bench.py, then this summary):",
        f"#   rocprofv3 --pmc FETCH_SIZE -d FETCH_DIR -o run --output-format csv -- python3 bench.py --steps 4 --warmup 1 --no-cpu-baseline{flag}",
        f"#   rocprofv3 --pmc WRITE_SIZE -d WRITE_DIR -o run --output-format csv -- python3 bench.py --steps 4 --warmup 1 --no-cpu-baseline{flag}",
        f"#   python3 bench.py --traffic-from FETCH_DIR WRITE_DIR{flag}",
        f"copy_kernel_bytes: {COPY_BYTES}  (read, and again written, by nkv_copy_bytes)",
        f"copy_kernel_FETCH_SIZE_KiB: {fetch[COPY_KERNEL]:.1f}  -> fetch scale {f_scale:.4f}",
        f"copy_kernel_WRITE_SIZE_KiB: {write[COPY_KERNEL]:.1f}  -> write scale {w_scale:.4f}",
        f"prefix_kernel_FETCH_SIZE_KiB: {fetch[PREFIX_KERNEL]:.1f}  -> {f_bytes:.0f} B",
        f"prefix_kernel_WRITE_SIZE_KiB: {write[PREFIX_KERNEL]:.1f}  -> {w_bytes:.0f} B",
        f"algorithmic_bytes_per_launch: {alg}",
        f"traffic_bytes_per_launch: {f_bytes + w_bytes:.0f}",
        f"traffic_over_algorithmic: {(f_bytes + w_bytes) / alg:.4f}",
    ]
    if "attn_tail_kernel" in fetch and "attn_tail_kernel" in write:
        lines.append(f"tail_kernel_traffic_bytes_per_launch: "
                     f"{fetch['attn_tail_kernel'] * 1024 * f_scale + write['attn_tail_kernel'] * 1024 * w_scale:.0f}")
    (TRAFFIC_FILE_TOK if tok else TRAFFIC_FILE).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def read_traffic(path: Path = TRAFFIC_FILE):
    """HBM bytes per launch of the prefix kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), or None."""
    if not path.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(budget_s: float, scheme: str = "t64") -> dict:
    """Time the numpy oracle's decode step for one layer at 32k context: dequantize the
    int8 prefix with the stored rulers, softmax attention over prefix + ring. Threads run
    the 8 KV heads in parallel (numpy releases the GIL inside its kernels)."""
    import numpy as np

    from oracle import attn as oattn
    from oracle import kvquant as okq

    rng = np.random.default_rng(0)
    n = CTX
    k = rng.standard_normal((HKV, n, D), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((HKV, n, D), dtype=np.float32).astype(np.float16)
    tok = scheme == "tok"
    if tok:
        kq, ks = okq.quantize_tok(k)
        vq, vs = okq.quantize_tok(v)
    else:
        kq, kmn, kst = okq.quantize_int8_token(k, 64)
        vq, vmn, vst = okq.quantize_int8_token(v, 64)
    ring_k = k[:, -64:].copy()
    ring_v = v[:, -64:].copy()
    q = (rng.standard_normal((HQ, D)) / D ** 0.5).astype(np.float16)
    gq = HQ // HKV
    threads = min(HKV, os.cpu_count() or 1)

    def head(h):
        if tok:
            k16 = okq.dequantize_tok(kq[h], ks[h])
            v16 = okq.dequantize_tok(vq[h], vs[h])
        else:
            k16 = okq.dequantize_int8_token(kq[h:h + 1], kmn[h:h + 1], kst[h:h + 1], 64)[0]
            v16 = okq.dequantize_int8_token(vq[h:h + 1], vmn[h:h + 1], vst[h:h + 1], 64)[0]
        kk = np.concatenate([k16, ring_k[h, :1]], 0)
        vv = np.concatenate([v16, ring_v[h, :1]], 0)
        return oattn.attend_fp16_kv(q[h * gq:(h + 1) * gq], kk[None], vv[None])[0]

    reps = 0
    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        while True:
            list(ex.map(head, range(HKV)))
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or (reps >= 3 and el > budget_s * 0.7):
                break
    per_layer = el / reps
    per_step = per_layer * LAYERS
    return {"value": 1.0 / per_step, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"numpy oracle ({scheme}), 1 layer x {reps} decode steps at {CTX} ctx ({el:.1f} s), "
                      f"scaled x{LAYERS} layers (extrapolated)",
            "seconds_per_step": per_step}


COPY_BYTES = 64 << 20


MFMA_FP16_PEAK_TFLOPS = 2500.0


def bench_prefill(args) -> int:
    """Chunked prefill over int8 KV: a 512-token fp16 query chunk attending causally to a
    16384-token int8t64 cache plus itself, 32 q / 8 KV heads, head_dim 128 (seed 4). Timed
    with HIP events over K graph replays of the two launches. Prints one JSON line: chunks/s,
    achieved TFLOP/s and MFMA utilisation (against the dense fp16 peak), GB/s."""
    import torch

    from nova_amd import _lib
    from nova_amd.kvattn import int8_prefill_attend, pack_int8_kv

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    M, U = 512, 16384
    K = args.steps if args.steps != 256 else 64
    W = args.warmup
    g = torch.Generator(device=dev).manual_seed(4)
    k = torch.randn(1, HKV, U, D, generator=g, device=dev).half()
    v = torch.randn(1, HKV, U, D, generator=g, device=dev).half()
    packed = [t.contiguous() for t in pack_int8_kv(k, v)]
    del k, v
    q = torch.randn(1, HQ, M, D, generator=g, device=dev).half()
    kc = torch.randn(1, HKV, M, D, generator=g, device=dev).half()
    vc = torch.randn(1, HKV, M, D, generator=g, device=dev).half()
    out = torch.empty_like(q)
    splits = args.splits or int(_lib.load().nkv_prefill_default_splits(HKV, HQ, M, U))
    scratch = torch.empty(int(_lib.load().nkv_prefill_workspace_bytes(HKV, HQ, M, splits)), dtype=torch.uint8, device=dev)
    int8_prefill_attend(q, kc, vc, *packed, used=U, out=out, scratch=scratch, splits=splits)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        int8_prefill_attend(q, kc, vc, *packed, used=U, out=out, scratch=scratch, splits=splits)
    stream = torch.cuda.current_stream(dev)
    for _ in range(W):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(K):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / K
    assert torch.isfinite(out).all()
    flop = 2 * 2 * D * HQ * (M * U + M * (M + 1) // 2)
    nbytes = U * 2176 + 2 * M * HQ * D * 2 + 2 * M * HKV * D * 2  # codes + rulers, q + out, chunk K/V
    tflops = flop / (ms / 1e3) / 1e12
    res = {
        "metric": "chunked-prefill attention over int8 KV: chunks/s, TFLOP/s, MFMA utilisation, GB/s",
        "value": round(1e3 / ms, 2), "unit": "chunks/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"{M}-token fp16 chunk causally over a {U}-token int8t64 cache plus itself, "
                               "32 q / 8 kv heads, head_dim 128", "chunk": M, "cache_tokens": U, "splits": splits},
        "flop_per_step": flop,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4), "traffic": None},
        "gbs": round(nbytes / (ms / 1e3) / 1e9, 1),
    }
    print(json.dumps(res), flush=True)
    return 0


VOCAB_QWEN3_4B = 151936


def cpu_baseline_e2e(budget_s: float, layer_shapes: list, lm_shape: tuple) -> dict:
    """The decode step of the random-weight decoder on the host: one layer's projections as
    fp32 torch matrix-vector products (all host threads) plus the numpy oracle's attention for
    one layer at 32k context, scaled to 36 layers, plus the lm_head product."""
    import torch

    att = cpu_baseline(budget_s * 0.6, "t64")
    per_layer_attn = att["seconds_per_step"] / LAYERS
    g = torch.Generator().manual_seed(0)
    ws = [torch.randn(*shp, generator=g) for shp in layer_shapes]
    lm = torch.randn(*lm_shape, generator=g)

    def run(mats):
        for w in mats:
            torch.mv(w, torch.ones(w.shape[1]))

    reps, t0 = 0, time.perf_counter()
    while True:
        run(ws)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s * 0.3 or reps >= 50:
            break
    per_layer_mv = el / reps
    t1 = time.perf_counter()
    run([lm])
    lm_s = time.perf_counter() - t1
    per_step = LAYERS * (per_layer_mv + per_layer_attn) + lm_s
    return {"value": 1.0 / per_step, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"one layer's projections as fp32 torch.mv ({reps} reps, {torch.get_num_threads()} threads) "
                      f"+ {att['sample']} + the lm_head product once; scaled to {LAYERS} layers (extrapolated)"}


def bench_e2e(args) -> int:
    """End-to-end graph decode of the random-weight decoder with Qwen3-4B geometry (36 layers,
    hidden 2560, 32 q / 8 KV heads of 128, SwiGLU 9728, vocab 151936, fp16 weights ~ N(0, 1/fan_in))
    over the int8t64 KV cache: the prompt (seeded random ids, ``--ctx`` tokens) is prefilled in
    streamed chunks, then each decode step (embed, 36 x [qkv GEMV + RMSNorm, q/k norm + RoPE,
    fused int8 append + attention, o_proj + residual, SwiGLU gate/up + RMSNorm, down + residual],
    final RMSNorm + lm_head, argmax, pos += 1) is one hipGraph replay. Each kernel is also timed
    alone (a graph of its 36 launches per step with the same weights); ``roofline`` is the one
    that takes the most time per step."""
    import torch

    from nova_amd import _lib
    from nova_amd import gemv as G
    from nova_amd.decode import GraphDecoder
    from nova_amd.skeleton import SkeletonConfig, SkeletonForCausalLM

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L, ctx, W = args.layers, args.ctx, args.warmup
    K = args.steps
    cfg = SkeletonConfig(num_hidden_layers=L, vocab_size=VOCAB_QWEN3_4B)
    model = SkeletonForCausalLM(cfg, seed=5, device=dev, dtype=torch.float16).eval()
    model.use_decode_kernels(True)
    max_len = -(-(ctx + 4 + W + K + 1) // 64) * 64
    dec = GraphDecoder(model, max_len=max_len, quant="int8", device=dev)
    if args.parts:
        dec.cache.set_parts(args.parts)
    ids = torch.randint(0, cfg.vocab_size, (1, ctx), generator=torch.Generator().manual_seed(6)).to(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.prefill(ids, chunk=args.chunk)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    dec.capture(warmup=3)
    stream = torch.cuda.current_stream(dev)
    for _ in range(W):
        dec.step()
    torch.cuda.synchronize()
    pos0 = int(dec.cache.pos.item())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        dec.step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = e0.elapsed_time(e1)
    assert int(dec.cache.pos.item()) == pos0 + K
    assert torch.isfinite(dec.logits).all()

    # ---- algorithmic bytes of one step: every weight once, the attention's KV bytes, the append
    layers = model.model.layers
    lay0 = layers[0]
    hid, inter = cfg.hidden_size, cfg.intermediate_size
    w_layer = sum(t.numel() * 2 for t in (lay0.w_qkv, lay0.attn.o_proj.weight, lay0.w_gate_up,
                                          lay0.mlp.down_proj.weight, lay0.norm, lay0.post_norm,
                                          lay0.attn.q_norm, lay0.attn.k_norm))
    w_head = model.lm_head.weight.numel() * 2 + hid * 2 + hid * 2  # lm_head, final norm, embedding row
    us = [pos0 + i + 1 for i in range(K)]
    kv_step = sum(attn_bytes(u) + APPEND_BYTES for u in us) / K * L
    step_bytes = L * w_layer + w_head + kv_step

    # ---- each kernel alone: a graph of its launches for one step, K replays
    gen = torch.Generator(device=dev).manual_seed(7)
    xh = torch.randn(hid, generator=gen, device=dev).half()
    xa = torch.randn(cfg.num_attention_heads * cfg.head_dim, generator=gen, device=dev).half()
    xi = torch.randn(inter, generator=gen, device=dev).half()
    res = torch.randn(hid, generator=gen, device=dev).half()
    o_h = torch.empty(hid, dtype=torch.float16, device=dev)
    o_qkv = torch.empty(lay0.w_qkv.shape[0], dtype=torch.float16, device=dev)
    o_i = torch.empty(inter, dtype=torch.float16, device=dev)
    o_v = torch.empty(cfg.vocab_size, dtype=torch.float16, device=dev)
    qkv = torch.randn(lay0.w_qkv.shape[0], generator=gen, device=dev).half()
    pos = dec.cache.pos
    inv = model.model.inv_freq32
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim

    def graph_of(fn, reps=1):
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        return g

    def time_graph(g) -> float:
        for _ in range(W):
            g.replay()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(K):
            g.replay()
        s1.record(stream)
        torch.cuda.synchronize()
        return s0.elapsed_time(s1)

    kv_in = torch.randn(2, 1, hkv, 1, d, generator=gen, device=dev).half()
    q_in = (torch.randn(1, hq, 1, d, generator=gen, device=dev) / d ** 0.5).half()
    kernels = {
        "nkv_gemv qkv+RMSNorm": (lambda: [G.rms_gemv(xh, ly.w_qkv, ly.norm, cfg.rms_eps, out=o_qkv) for ly in layers],
                                 lay0.w_qkv.numel() * 2, L),
        "nkv_qk_norm_rope": (lambda: [G.qk_norm_rope_(qkv, hq, hkv, ly.attn.q_norm, ly.attn.k_norm, cfg.rms_eps, inv, pos)
                                      for ly in layers], (hq + hkv) * d * 4, L),
        "nkv_decode_step_t64": (lambda: [dec.cache.update_attend(kv_in[0], kv_in[1], q_in, i) for i in range(L)],
                                sum(attn_bytes(u) + APPEND_BYTES for u in us) / K, L),
        "nkv_gemv o_proj+residual": (lambda: [G.rms_gemv(xa, ly.attn.o_proj.weight, residual=res, out=o_h)
                                              for ly in layers], ly_bytes(lay0.attn.o_proj.weight), L),
        "nkv_swiglu_gemv gate/up+RMSNorm": (lambda: [G.swiglu_gemv(xh, ly.w_gate_up, ly.post_norm, cfg.rms_eps, out=o_i)
                                                     for ly in layers], ly_bytes(lay0.w_gate_up), L),
        "nkv_gemv down+residual": (lambda: [G.rms_gemv(xi, ly.mlp.down_proj.weight, residual=res, out=o_h)
                                            for ly in layers], ly_bytes(lay0.mlp.down_proj.weight), L),
        "nkv_gemv lm_head+RMSNorm": (lambda: G.rms_gemv(xh, model.lm_head.weight, model.model.norm, cfg.rms_eps,
                                                        out=o_v), ly_bytes(model.lm_head.weight), 1),
    }
    saved = dec._save_int8_state()
    breakdown = {}
    for name, (fn, nbytes, launches) in kernels.items():
        with torch.inference_mode():  # the decoder's state tensors are inference tensors
            g = graph_of(fn)
            t = time_graph(g) / K  # ms per step
        del g
        per_launch = t / launches / 1e3
        breakdown[name] = {"launches_per_step": launches, "ms_per_step": round(t, 4),
                           "avg_launch_us": round(per_launch * 1e6, 3),
                           "algorithmic_bytes_per_launch": round(nbytes),
                           "gbs": round(nbytes / per_launch / 1e9, 1)}
    dec._restore_int8_state(saved)
    top = max(breakdown, key=lambda n: breakdown[n]["ms_per_step"])
    tb = breakdown[top]

    ms_step = ms / K
    out = {
        "metric": "end-to-end graph-decode tokens/s, 36-layer Qwen3-4B-geometry decoder (random weights) "
                  "over the int8 KV cache at 32k ctx",
        "value": round(K / (ms / 1e3), 2), "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (random weights, random prompt ids)",
        "config": {"workload": f"greedy decode, {L} layers x (hidden {hid}, 32 q / 8 kv heads x 128, SwiGLU {inter}), "
                               f"vocab {cfg.vocab_size}, batch 1, int8t64 KV cache, {ctx}-token prompt prefilled in "
                               f"{args.chunk}-token streamed chunks, {K} hipGraph-replayed steps",
                   "layers": L, "context": ctx, "hidden": hid, "intermediate": inter, "vocab": cfg.vocab_size,
                   "prefill_chunk": args.chunk, "parts_per_head": dec.cache._n_parts},
        "algorithmic_bytes_per_step": round(step_bytes),
        "step_gbs": round(step_bytes / (ms_step / 1e3) / 1e9, 1),
        "step_pct_of_hbm_peak": round(100 * step_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
        "prefill_s": round(prefill_s, 3),
        "prefill_tokens_per_s": round(ctx / prefill_s, 1),
        "wall_s_timed": round(wall, 4),
        "roofline": {"bound": "hbm", "achieved": tb["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(tb["gbs"] / HBM_PEAK_GBS, 4), "traffic": None, "kernel": top,
                     "algorithmic_bytes_per_launch": tb["algorithmic_bytes_per_launch"],
                     "avg_launch_us": tb["avg_launch_us"]},
        "kernels": breakdown,
        "kernels_sum_ms_per_step": round(sum(b["ms_per_step"] for b in breakdown.values()), 4),
    }
    if not args.no_cpu_baseline:
        shapes = [tuple(t.shape) for t in (lay0.w_qkv, lay0.attn.o_proj.weight, lay0.w_gate_up,
                                           lay0.mlp.down_proj.weight)]
        out["cpu_baseline"] = cpu_baseline_e2e(args.cpu_seconds, shapes, tuple(model.lm_head.weight.shape))
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


def ly_bytes(w) -> int:
    return w.numel() * 2


def bench_paged(args) -> int:
    """Batched ragged decode: 8 sequences with seeded uniform lengths in [1024, 16384]
    (seed 3), 36 layers, int8t64 pages of 64 tokens; one step = every layer's
    append + attention for all 8 sequences, captured as one hipGraph. Prints one JSON line
    (batch tokens/s; GB/s over the algorithmic bytes of the valid tokens, padding excluded)."""
    import torch

    from nova_amd import _lib
    from nova_amd.paged import PagedKVInt8Cache

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L, B = args.layers, 8
    K = args.steps if args.steps != 256 else 128
    W = args.warmup
    gen = torch.Generator().manual_seed(3)
    lens = [int(x) for x in torch.randint(1024, 16385, (B,), generator=gen)]
    per_seq = max(-(-(n + W + K + 2) // 64) for n in lens)
    total_pages = sum(-(-(n + W + K + 2) // 64) for n in lens)
    cache = PagedKVInt8Cache(L, HKV, D, HQ, max_seqs=B, num_pages=total_pages, max_pages_per_seq=per_seq, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    for b, n in enumerate(lens):
        cache.reserve(b, n + W + K + 1)
        for layer in range(L):
            k = torch.randn(1, HKV, n, D, generator=g, device=dev).half()
            v = torch.randn(1, HKV, n, D, generator=g, device=dev).half()
            cache.prefill(b, layer, k, v)
    cache.plan()
    torch.cuda.synchronize()
    qs = [(torch.randn(B, HQ, 1, D, generator=g, device=dev) / D ** 0.5).half() for _ in range(L)]
    ks = [torch.randn(B, HKV, 1, D, generator=g, device=dev).half() for _ in range(L)]
    vs = [torch.randn(B, HKV, 1, D, generator=g, device=dev).half() for _ in range(L)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for layer in range(L):
            cache.decode_step(ks[layer], vs[layer], qs[layer], layer)
        cache.pos[:B].add_(1)
    stream = torch.cuda.current_stream(dev)
    for _ in range(W):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = e0.elapsed_time(e1)
    assert torch.isfinite(cache.merged[:B]).all()
    step_bytes = sum(sum(attn_bytes(n + W + i + 1) + APPEND_BYTES for n in lens) for i in range(K)) / K * L
    ms_step = ms / K
    gbs = step_bytes / (ms_step / 1e3) / 1e9
    out = {
        "metric": "paged ragged batch int8-KV decode: batch tokens/s + achieved HBM GB/s (% of peak)",
        "value": round(B * K / (ms / 1e3), 2),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"paged int8t64 decode, {B} ragged sequences (lengths {lens}), {L} layers x "
                               "(32 q / 8 kv heads, head_dim 128), 64-token pages, hipGraph-replayed steps",
                   "lengths": lens, "layers": L, "page_tokens": 64, "work_units_per_head": cache.total_parts},
        "step_gbs": round(gbs, 1),
        "step_pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "algorithmic_bytes_per_step": round(step_bytes),
        "wall_s_timed": round(wall, 4),
    }
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    if args.traffic_from:
        write_traffic(*args.traffic_from, scheme=args.scheme)
        return 0
    if args.workload == "paged" and args.gpus == 1:
        return bench_paged(args)
    if args.workload == "prefill" and args.gpus == 1:
        return bench_prefill(args)
    if args.workload == "e2e" and args.gpus == 1:
        return bench_e2e(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported on this path "
              "(the decode attention shards by KV head across GPUs; see the design notes)", file=sys.stderr)
        return 2

    import torch

    from nova_amd import _lib
    from nova_amd.kvattn import KVInt8Cache
    from nova_amd.kvtok import KVInt8TokCache

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L, ctx, W, K = args.layers, args.ctx, args.warmup, args.steps
    max_len = -(-(ctx + 3 * (W + K) + 1) // 64) * 64

    # ---- prefill: seeded N(0,1) K/V, 4 random K channels per head x8, quantized by the
    # bulk HIP quantizer into the cache (staging area -> finish_prefill)
    tok = args.scheme == "tok"
    cls = KVInt8TokCache if tok else KVInt8Cache
    cache = cls(num_slots=L, num_kv_heads=HKV, head_dim=D, max_len=max_len, num_q_heads=HQ, device=dev)
    if args.parts:
        cache.set_parts(args.parts)
    gen = torch.Generator(device=dev).manual_seed(2)
    cpu_gen = torch.Generator().manual_seed(3)
    cache.begin_prefill(ctx)
    cache.set_prefill_pos(0)
    for layer in range(L):
        k = torch.randn(1, HKV, ctx, D, generator=gen, device=dev)
        for h in range(HKV):
            ch = torch.randperm(D, generator=cpu_gen)[:4].to(dev)
            k[0, h, :, ch] *= 8.0
        v = torch.randn(1, HKV, ctx, D, generator=gen, device=dev)
        cache.update(k.half(), v.half(), layer)
        del k, v
    cache.finish_prefill(ctx)
    torch.cuda.synchronize()

    # ---- per-layer synthetic decode inputs (q ~ N(0,1)/sqrt(128))
    qs = [(torch.randn(1, HQ, 1, D, generator=gen, device=dev) / D ** 0.5).half() for _ in range(L)]
    ks = [torch.randn(1, HKV, 1, D, generator=gen, device=dev).half() for _ in range(L)]
    vs = [torch.randn(1, HKV, 1, D, generator=gen, device=dev).half() for _ in range(L)]

    def step():
        for layer in range(L):
            cache.update_attend(ks[layer], vs[layer], qs[layer], layer)
        cache.pos.add_(1)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    stream = torch.cuda.current_stream(dev)
    for _ in range(W):
        graph.replay()
    torch.cuda.synchronize()
    pos0 = int(cache.pos.item())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = e0.elapsed_time(e1)
    assert int(cache.pos.item()) == pos0 + K
    assert torch.isfinite(cache.merged).all()

    # ---- each of the step's two kernels alone: a graph of its 36 launches per step (the
    # same kernel and arguments as above), K replays timed with HIP events
    def kernel_graph(entry: str, advance: bool):
        args_per_layer = [cache.step_args(ks[layer], vs[layer], qs[layer], layer) for layer in range(L)]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for a in args_per_layer:
                _lib.call(entry, *a[:-1], _lib.stream_ptr(dev))
            if advance:
                cache.pos.add_(1)
        return g, args_per_layer

    def time_graph(g) -> float:
        for _ in range(W):
            g.replay()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(K):
            g.replay()
        s1.record(stream)
        torch.cuda.synchronize()
        return s0.elapsed_time(s1)

    sfx = "tok" if tok else "t64"
    g_prefix, keep = kernel_graph(f"nkv_decode_step_partials_{sfx}", True)
    pos_a = int(cache.pos.item()) + W
    ms_prefix = time_graph(g_prefix)
    g_tail, keep2 = kernel_graph(f"nkv_decode_step_combine_{sfx}", False)
    ms_tail = time_graph(g_tail)
    del keep, keep2

    # ---- traffic calibration copy (known byte count; read by the --pmc runs)
    cal = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
    cal2 = torch.empty_like(cal)
    _lib.call("nkv_copy_bytes", cal.data_ptr(), cal2.data_ptr(), cal.numel(), _lib.stream_ptr(dev))
    torch.cuda.synchronize()

    ms_step = ms / K
    tok_s = K / (ms / 1e3)
    us = [pos0 + i + 1 for i in range(K)]  # tokens written when each timed step attends
    if tok:
        step_bytes = sum(attn_bytes_tok(u) + APPEND_BYTES_TOK for u in us) / K * L
    else:
        step_bytes = sum(attn_bytes(u) + APPEND_BYTES for u in us) / K * L
    ua = [pos_a + i + 1 for i in range(K)]  # the same for the prefix-kernel graph's replays
    launch_bytes = sum((prefix_launch_bytes_tok if tok else prefix_launch_bytes)(u) for u in ua) / K
    per_launch_s = ms_prefix / 1e3 / (K * L)
    achieved = launch_bytes / per_launch_s / 1e9
    traffic = read_traffic(TRAFFIC_FILE_TOK if tok else TRAFFIC_FILE)
    out = {
        "metric": "int8-KV decode attention tokens/s + achieved HBM GB/s (% of peak) at 32k ctx",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": f"{'per-token symmetric int8' if tok else 'int8t64'} KV decode step, {L} layers x "
                        f"(32 q / 8 kv heads, head_dim 128), batch 1, "
                        f"{ctx}-token prefilled cache, {K} hipGraph-replayed steps",
            "layers": L, "context": ctx, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "batch": 1,
            "kv_format": ("tok (int8 codes, one fp16 absmax scale per token and KV head)" if tok
                          else "int8t64 (uint8 codes, fp16 min/step per 64 tokens per channel)"),
            "parts_per_head": cache._n_parts,
        },
        "step_gbs": round(step_bytes / (ms_step / 1e3) / 1e9, 1),
        "step_pct_of_hbm_peak": round(100 * step_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
        "wall_s_timed": round(wall, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": f"nkv::attn_prefix_kernel<{'true' if tok else 'false'}> (append + split-K partials over the int8 prefix)",
            "algorithmic_bytes_per_launch": round(launch_bytes),
            "avg_launch_us": round(per_launch_s * 1e6, 3),
        },
        "tail_kernel": {
            "kernel": "nkv::attn_tail_kernel (ring attention + log-sum-exp combine)",
            "avg_launch_us": round(ms_tail / (K * L) * 1e3, 3),
        },
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline(args.cpu_seconds, args.scheme)
        cb.pop("seconds_per_step")
        out["cpu_baseline"] = cb
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
