"""Benchmark: int8-KV decode attention over 36 layers at 32k context on one MI355X.

Headline workload (the long-context decode configuration): 36 layers x (32 q heads, 8 KV heads,
head_dim 128), batch 1, int8t64 KV cache prefilled to 32768 tokens from seeded N(0,1) fp16 K/V
with 4 random K channels per head scaled x8. One decode step = every layer's append + attention
in one chained launch (``ChainedStep``, ``nkv_decode_layers_t64``), then ``pos += 1``. The
layers are chained as in a model: layer l's query and its new K/V token are views of layer l-1's
attention output (q = the whole output, k = q heads 0, 4, .., v = q heads 1, 5, ..; layer 0 reads
the previous step's last output), and with the default ``--dep all`` no input of layer l is read
before every KV head of layer l-1 has finished (the all-head dependency of a model, where every
q head of layer l depends on every head of layer l-1 through o_proj). The step is captured once
as a hipGraph; SETTLE_STEPS + W untimed replays (the first SETTLE_STEPS let the clocks reach their
steady state), then K timed replays bracketed by ``torch.cuda.synchronize()``
and HIP events on the replay stream; afterwards the launch's error word is checked.

One JSON line (the driver's contract). ``value`` = decode tokens/s of the whole job.
``roofline`` is the chained launch: algorithmic bytes per launch / its average duration, timed
with HIP events over K replays of a graph of the launch alone. ``traffic`` comes from the
committed rocprofv3 --pmc summary of that kernel (FETCH_SIZE + WRITE_SIZE per dispatch, each
scaled by what the counter reads for the library's copy kernel of known size). ``cpu_baseline``
times the repo's torch fp32 restatement of the reference algorithm (dequantize the int8 prefix,
append the ring, repeat KV heads, softmax attention) on the host cores for one layer and a few
steps, scaled to the 36-layer step. ``core_clock`` is each XCD's core clock right after the timed
replays, from the device's core and 100 MHz real-time counters (``nkv_clock_probe``);
``gpu_clock`` is what amd-smi reports while the launches replay (on some hosts it reports an
idle clock under load). ``workloads`` carries the other configurations measured in the same run: the per-head
dependency, one launch per layer (what a model's layer loop calls), the per-token symmetric
format, the paged ragged batch, the MFMA chunked prefill, the read ceiling of the decode path's
load pattern and the end-to-end random-weight decoder.

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--no-cpu-baseline] [--only]
    python bench.py --workload decode|paged|prefill|e2e|read [--scheme t64|tok] [--mode chain|layers]
                    [--dep all|head]                                        # one workload alone
    python bench.py --traffic-from FETCH_DIR WRITE_DIR --traffic-key KEY    # summarize --pmc runs
    python bench.py --stats-from OUT_DIR --stats-name NAME --stats-cmd CMD  # summarize a --stats run
"""

from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import threading
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

LAYERS, HQ, HKV, D, CTX = 36, 32, 8, 128, 32768
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
COPY_BYTES = 64 << 20
# the int8t64 append per layer and step: K and V rings read (64 x 128 fp16 per KV head), the new
# token read and written into the ring, 64 code rows and 4 ruler rows written
APPEND_BYTES = 64 * 128 * 2 * 2 * HKV + 2 * 2 * 128 * 2 * HKV + 64 * 128 * 2 * HKV + 4 * 128 * 2 * HKV
# the per-token symmetric append: the new token read, its codes and scale written
APPEND_BYTES_TOK = 2 * 128 * 2 * HKV + 2 * 128 * HKV + 2 * 2 * HKV
COPY_KERNEL = "copy16_kernel"
PROFILES = ROOT / "profiles"
# traffic summaries: key -> (file, the kernel's name in rocprof's CSV, the command profiled)
_DEC = "python3 bench.py --workload decode --steps 4 --warmup 1 --no-cpu-baseline --no-clock"
TRAFFIC = {
    "chain_t64": (PROFILES / "decode_chain_32k_traffic.txt", "attn_layers_kernel<0>", _DEC + " --mode chain"),
    "chain_tok": (PROFILES / "decode_chain_tok_32k_traffic.txt", "attn_layers_kernel<1>",
                  _DEC + " --mode chain --scheme tok"),
    "layers_t64": (PROFILES / "decode_step_32k_traffic.txt", "attn_prefix_kernel<0, false>", _DEC + " --mode layers"),
    "layers_tok": (PROFILES / "decode_step_tok_32k_traffic.txt", "attn_prefix_kernel<1, false>",
                   _DEC + " --mode layers --scheme tok"),
    "paged_t64": (PROFILES / "paged_batch_decode_traffic.txt", "attn_prefix_kernel<2, false>",
                  "python3 bench.py --workload paged --steps 4 --warmup 1 --no-clock"),
    "paged_tok": (PROFILES / "paged_batch_decode_tok_traffic.txt", "attn_prefix_kernel<3, false>",
                  "python3 bench.py --workload paged --scheme tok --steps 4 --warmup 1 --no-clock"),
    "prefill": (PROFILES / "prefill_chunk_512_over_16k_traffic.txt", "prefill_chunk_kernel",
                "python3 bench.py --workload prefill --steps 4 --warmup 1 --no-clock"),
}
VOCAB_QWEN3_4B = 151936
# Untimed step replays before the W warmup steps of a decode measurement: after the prefill and the
# graph capture the GPU's clocks ramp up over the first few dozen steps (with 5 warmup steps the
# timed 20 ran 9% slower than with 60), so the timed steps are taken at the steady state.
SETTLE_STEPS = 128


def attn_bytes(u: int) -> int:
    """Algorithmic bytes of one layer's int8t64 decode attention with ``u`` tokens written:
    codes + fp16 rulers of the whole groups (2176 B per token over 8 KV heads), the fp16 ring
    tokens (4096 B each), q and out (16384 B)."""
    q = u // 64 * 64
    return 2176 * q + 4096 * (u - q) + 16384


def attn_bytes_tok(u: int) -> int:
    """The same for the per-token symmetric format: int8 codes + one fp16 scale per token, K and
    V, 8 KV heads (2080 B per token), q and out."""
    return 2080 * u + 16384


def step_launch_bytes(u: int, scheme: str = "t64") -> int:
    """Algorithmic bytes of one fused decode-step launch (append + attention) at ``u`` tokens
    written after the append."""
    return attn_bytes_tok(u) + APPEND_BYTES_TOK if scheme == "tok" else attn_bytes(u) + APPEND_BYTES


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
    ap.add_argument("--only", action="store_true", help="the headline workload alone (no extra workloads)")
    ap.add_argument("--no-clock", action="store_true", help="skip the amd-smi clock reading")
    ap.add_argument("--chunk", type=int, default=2048, help="e2e: streamed prefill chunk (a multiple of 64)")
    ap.add_argument("--workload", choices=("decode", "paged", "prefill", "e2e", "read"), default=None,
                    help="run one workload alone and print its line")
    ap.add_argument("--scheme", choices=("t64", "tok"), default="t64",
                    help="--workload decode: KV format, int8t64 (the reference's) or per-token symmetric")
    ap.add_argument("--mode", choices=("chain", "layers"), default="chain",
                    help="--workload decode: every layer in one launch (chain) or one launch per layer")
    ap.add_argument("--dep", choices=("all", "head"), default="all",
                    help="--mode chain: every layer waits for every head of the layer before (all), or forwarded "
                         "inputs wait only for their own head (head)")
    ap.add_argument("--e2e-steps", type=int, default=32, help="steps of the end-to-end workload in the default run")
    ap.add_argument("--e2e-separate", action="store_true",
                    help="e2e: the attention block as three launches (qkv GEMV, q/k norm + RoPE, decode step)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarize two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) into a traffic file")
    ap.add_argument("--traffic-key", choices=sorted(TRAFFIC), default="chain_t64")
    ap.add_argument("--stats-from", metavar="OUT_DIR", help="summarize a rocprofv3 --kernel-trace --stats run")
    ap.add_argument("--stats-name", help="--stats-from: the summary's file name under profiles/")
    ap.add_argument("--stats-cmd", help="--stats-from / --counters-from: the command that was profiled")
    ap.add_argument("--counters-from", nargs="+", metavar="OUT_DIR",
                    help="summarize rocprofv3 --pmc runs (one per counter set) of one kernel")
    ap.add_argument("--counters-kernel", help="--counters-from: the kernel's name (a substring)")
    ap.add_argument("--counters-name", help="--counters-from: the summary's file name under profiles/")
    return ap.parse_args()


# ---------------------------------------------------------------- rocprof traffic summaries


def _pmc_means(run_dir: str, counter: str, kernel: str) -> dict:
    """Mean per-dispatch value of ``counter`` per kernel (``kernel``, the copy kernel) in a
    rocprofv3 --pmc CSV run."""
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
                for key in (kernel, COPY_KERNEL):
                    if key in row["Kernel_Name"]:
                        acc.setdefault(key, []).append(float(row["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def write_traffic(fetch_dir: str, write_dir: str, key: str) -> None:
    """HBM bytes per dispatch of the workload's dominant kernel from FETCH_SIZE and WRITE_SIZE
    (KiB), each scaled by the factor that makes the same counter read the copy kernel's known
    bytes."""
    path, kernel, cmd = TRAFFIC[key]
    fetch, write = _pmc_means(fetch_dir, "FETCH_SIZE", kernel), _pmc_means(write_dir, "WRITE_SIZE", kernel)
    f_scale = COPY_BYTES / (fetch[COPY_KERNEL] * 1024)
    w_scale = COPY_BYTES / (write[COPY_KERNEL] * 1024)
    f_bytes = fetch[kernel] * 1024 * f_scale
    w_bytes = write[kernel] * 1024 * w_scale
    lines = [
        f"# HBM traffic per dispatch of nkv::{kernel} ({key})",
        "# made by (two rocprofv3 --pmc runs of the workload, then this summary; from the repository root):",
        f"#   rocprofv3 --pmc FETCH_SIZE -d FETCH_DIR -o run --output-format csv -- {cmd}",
        f"#   rocprofv3 --pmc WRITE_SIZE -d WRITE_DIR -o run --output-format csv -- {cmd}",
        f"#   python3 bench.py --traffic-from FETCH_DIR WRITE_DIR --traffic-key {key}",
        f"copy_kernel_bytes: {COPY_BYTES}  (read, and again written, by nkv_copy_bytes)",
        f"copy_kernel_FETCH_SIZE_KiB: {fetch[COPY_KERNEL]:.1f}  -> fetch scale {f_scale:.4f}",
        f"copy_kernel_WRITE_SIZE_KiB: {write[COPY_KERNEL]:.1f}  -> write scale {w_scale:.4f}",
        f"kernel_FETCH_SIZE_KiB: {fetch[kernel]:.1f}  -> {f_bytes:.0f} B",
        f"kernel_WRITE_SIZE_KiB: {write[kernel]:.1f}  -> {w_bytes:.0f} B",
        f"traffic_bytes_per_launch: {f_bytes + w_bytes:.0f}",
        "(bench.py divides this by its own algorithmic bytes per launch: roofline.traffic_over_algorithmic)",
    ]
    path.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def read_traffic(key: str):
    """HBM bytes per launch of a workload's dominant kernel from the committed summary, or None."""
    path = TRAFFIC[key][0]
    if not path.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text(), re.M)
    return float(m.group(1)) if m else None


def write_counters(dirs: list, kernel: str, name: str, cmd: str) -> None:
    """Per-dispatch means of every counter that rocprofv3 --pmc runs (one directory per counter
    set) recorded for ``kernel``, with the derived MFMA, VALU and LDS figures when their counters
    are present."""
    import csv

    acc: dict = {}
    sets = []
    for d in dirs:
        names = set()
        for f in sorted(Path(d).rglob("*counter_collection.csv")):
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    if kernel in row["Kernel_Name"]:
                        acc.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
                        names.add(row["Counter_Name"])
        sets.append(sorted(names))
    mean = {k: sum(v) / len(v) for k, v in acc.items()}
    lines = [f"# rocprofv3 counters of nkv::{kernel}, per dispatch (mean over the dispatches of each pass)",
             "# made by (from the repository root, one MI355X; one pass per counter set):"]
    lines += [f"#   rocprofv3 --pmc {' '.join(cs)} -d OUT{i + 1} -o run --output-format csv -- {cmd}"
              for i, cs in enumerate(sets)]
    lines.append(f"#   python3 bench.py --counters-from {' '.join(f'OUT{i + 1}' for i in range(len(sets)))} "
                 f"--counters-kernel '{kernel}' --counters-name {name} --stats-cmd '{cmd}'")
    lines += [f"{k:<28} {v:>14.4g}" for k, v in sorted(mean.items())]
    der = []
    if "GRBM_GUI_ACTIVE" in mean:
        der.append(f"cycles per XCD: {mean['GRBM_GUI_ACTIVE'] / 8:.4g}")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and "GRBM_GUI_ACTIVE" in mean:
        der.append(f"MFMA pipe busy: {mean['SQ_VALU_MFMA_BUSY_CYCLES'] / 1024 / (mean['GRBM_GUI_ACTIVE'] / 8):.3f} of each "
                   "SIMD's cycles (SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / cycles per XCD)")
    if "SQ_INSTS_VALU" in mean and "SQ_INSTS_MFMA" in mean:
        der.append(f"VALU instructions per MFMA: {mean['SQ_INSTS_VALU'] / mean['SQ_INSTS_MFMA']:.2f}")
    if "SQ_INSTS_VALU" in mean and "GRBM_GUI_ACTIVE" in mean:
        der.append(f"VALU issue: {mean['SQ_INSTS_VALU'] / 1024 * 4 / (mean['GRBM_GUI_ACTIVE'] / 8):.3f} of each SIMD's "
                   "cycles (4 cycles per wave64 instruction)")
    if "SQ_LDS_BANK_CONFLICT" in mean and "SQ_LDS_IDX_ACTIVE" in mean:
        der.append(f"LDS bank-conflict share of LDS-active cycles: "
                   f"{mean['SQ_LDS_BANK_CONFLICT'] / mean['SQ_LDS_IDX_ACTIVE']:.3f}")
    if "SQ_LDS_IDX_ACTIVE" in mean and "GRBM_GUI_ACTIVE" in mean:
        der.append(f"LDS active: {mean['SQ_LDS_IDX_ACTIVE'] / 256 / (mean['GRBM_GUI_ACTIVE'] / 8):.3f} of each CU's cycles")
    if der:
        lines += ["# derived:"] + [f"#   {x}" for x in der]
    (PROFILES / name).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def write_stats(out_dir: str, name: str, cmd: str) -> None:
    """A short summary of a rocprofv3 --kernel-trace --stats run: per kernel the calls and the
    average, minimum, maximum and median duration, from the run's kernel trace."""
    import csv
    import statistics

    traces = sorted(Path(out_dir).rglob("*kernel_trace.csv"))
    if not traces:
        raise SystemExit(f"no kernel_trace.csv under {out_dir}")
    durs: dict = {}
    for f in traces:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                nm = row["Kernel_Name"]
                durs.setdefault(nm, []).append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    total = sum(sum(v) for v in durs.values())
    lines = [f"# rocprofv3 kernel trace summary ({name}); durations in ns",
             "# made by (from the repository root, one MI355X):",
             f"#   rocprofv3 --kernel-trace --stats -d OUT -o run --output-format csv -- {cmd}",
             f"#   python3 bench.py --stats-from OUT --stats-name {name} --stats-cmd '{cmd}'",
             f"{'kernel':<72} {'calls':>6} {'avg':>11} {'min':>9} {'max':>9} {'median':>11} {'share':>7}"]
    for nm, v in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
        short = re.sub(r"\(.*", "", nm.replace("void ", "").replace("(anonymous namespace)::", ""))[:72]
        lines.append(f"{short:<72} {len(v):>6} {sum(v) / len(v):>11.1f} {min(v):>9} {max(v):>9} "
                     f"{statistics.median(v):>11.1f} {100 * sum(v) / total:>6.2f}%")
    (PROFILES / name).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


# ---------------------------------------------------------------- host side: CPU baseline, clock


def host_threads() -> int:
    """The host threads this process may use: the CPUs it is pinned to, capped by OMP_NUM_THREADS."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s: float, scheme: str, ctx: int, layers: int) -> dict:
    """The reference algorithm on the host: the torch fp32 restatement (dequantize the int8
    prefix, append the valid ring slots, repeat the KV heads, softmax attention) of one layer's
    decode step at ``ctx`` tokens, timed over a few steps with every host thread, scaled to the
    ``layers``-layer step. The codes and rulers are synthetic (the timing does not depend on them)."""
    import torch

    from oracle import torch_ref

    torch.set_num_threads(host_threads())
    g = torch.Generator().manual_seed(0)
    q = (torch.randn(HQ, D, generator=g) / D ** 0.5).half()
    if scheme == "tok":
        kq = torch.randint(-127, 128, (HKV, ctx, D), generator=g, dtype=torch.int8)
        vq = torch.randint(-127, 128, (HKV, ctx, D), generator=g, dtype=torch.int8)
        ks = (torch.rand(HKV, ctx, generator=g) * 0.02 + 0.01).half()
        vs = (torch.rand(HKV, ctx, generator=g) * 0.02 + 0.01).half()
        run = lambda: torch_ref.decode_step_tok(q, kq, ks, vq, vs, ctx)  # noqa: E731
    else:
        ng = -(-ctx // 64)
        kq = torch.randint(0, 256, (HKV, ctx + 64, D), generator=g, dtype=torch.uint8)
        vq = torch.randint(0, 256, (HKV, ctx + 64, D), generator=g, dtype=torch.uint8)
        rul = [(torch.rand(HKV, ng + 1, D, generator=g) * s + o).half() for s, o in ((2, -3), (0.02, 0.01))] * 2
        ring_k = torch.randn(HKV, 64, D, generator=g).half()
        ring_v = torch.randn(HKV, 64, D, generator=g).half()
        written = ctx + 1  # the step after a 32768-token prefill: one token in the ring
        run = lambda: torch_ref.decode_step_t64(q, kq, rul[0], rul[1], vq, rul[2], rul[3], ring_k,  # noqa: E731
                                                ring_v, written)
    run()  # warm up
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 64:
            break
    per_step = el / reps * layers
    return {"value": round(1.0 / per_step, 4), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", "cpu_model": cpu_model(),
            "sample": f"torch fp32 restatement ({scheme}): 1 layer x {reps} decode steps at {ctx} ctx + ring "
                      f"({el:.1f} s, {torch.get_num_threads()} threads), scaled x{layers} layers (extrapolated)"}


def _walk_clocks(obj, path=""):
    """(path, MHz) of every ``{"clk": {"value": v}}``-like leaf of amd-smi's JSON."""
    if isinstance(obj, dict):
        for k, v in obj.items():
            p = f"{path}/{k}"
            if k in ("clk", "cur_clk", "current") and isinstance(v, dict) and "value" in v:
                try:
                    yield p, float(v["value"])
                except (TypeError, ValueError):
                    pass
            else:
                yield from _walk_clocks(v, p)
    elif isinstance(obj, list):
        for i, v in enumerate(obj):
            yield from _walk_clocks(v, f"{path}[{i}]")


def read_gpu_clock(timeout: float = 30.0) -> dict:
    """The GPU clocks as amd-smi reports them (``amd-smi metric --clock --json``)."""
    try:
        r = subprocess.run(["amd-smi", "metric", "--clock", "--json"], capture_output=True, text=True,
                           timeout=timeout)
    except (OSError, subprocess.TimeoutExpired) as e:
        return {"source": "amd-smi metric --clock", "error": str(e)[:200]}
    try:
        found = list(_walk_clocks(json.loads(r.stdout)))
    except ValueError:
        return {"source": "amd-smi metric --clock", "error": (r.stdout + r.stderr)[:300]}
    gfx = [v for p, v in found if "gfx" in p.lower()]
    mem = [v for p, v in found if "mem" in p.lower()]
    return {"source": "amd-smi metric --clock --json", "gfx_mhz": gfx[:8] or None, "mem_mhz": mem[:1] or None}


CLOCK_PROBE_WGS, CLOCK_PROBE_ITERS = 64, 20000  # ~70 us of one wave per workgroup


def core_clock(dev) -> dict:
    """Each XCD's core clock in MHz, from ``nkv_clock_probe`` launched now, right after a timed run
    (the clocks move over milliseconds, the probe takes ~70 us): per workgroup the core clock
    counter's advance (s_memtime) over the 100 MHz real-time counter's (s_memrealtime), averaged
    over the workgroups of each XCD."""
    import torch

    from nova_amd import _lib

    buf = torch.zeros(3 * CLOCK_PROBE_WGS, dtype=torch.int64, device=dev)
    _lib.call("nkv_clock_probe", buf.data_ptr(), CLOCK_PROBE_WGS, CLOCK_PROBE_ITERS, _lib.stream_ptr(dev))
    by_xcd: dict = {}
    for xcc, dm, dr in buf.view(CLOCK_PROBE_WGS, 3).cpu().tolist():
        if dr > 0:
            by_xcd.setdefault(int(xcc), []).append(100.0 * dm / dr)
    mhz = [round(sum(v) / len(v)) for _, v in sorted(by_xcd.items())]
    return {"source": "nkv_clock_probe: s_memtime over s_memrealtime (100 MHz), right after the timed replays",
            "gfx_mhz_by_xcd": mhz, "gfx_mhz_mean": round(sum(mhz) / len(mhz)) if mhz else None}


def clock_under_load(replay) -> dict:
    """Read the clock in a thread while ``replay()`` keeps the GPU busy (bounded to ~40 s)."""
    box: dict = {}
    t = threading.Thread(target=lambda: box.update(read_gpu_clock()), daemon=True)
    t.start()
    t0 = time.perf_counter()
    while t.is_alive() and time.perf_counter() - t0 < 40.0:
        replay()
    t.join(timeout=1.0)
    return box or {"source": "amd-smi metric --clock", "error": "no reading"}


# ---------------------------------------------------------------- the decode workloads


def _time_graph(graph, stream, reps: int, warmup: int, settle: int = 0) -> float:
    """ms per replay of ``graph`` over ``reps`` replays after ``settle + warmup`` untimed ones, HIP
    events on ``stream``."""
    import torch

    for _ in range(settle + warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _calibration_copy(dev) -> None:
    """One launch of the library's copy kernel over a known byte count: the --pmc runs scale
    FETCH_SIZE and WRITE_SIZE by what they read for it."""
    import torch

    from nova_amd import _lib

    cal = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
    cal2 = torch.empty_like(cal)
    _lib.call("nkv_copy_bytes", cal.data_ptr(), cal2.data_ptr(), cal.numel(), _lib.stream_ptr(dev))
    torch.cuda.synchronize()
    del cal, cal2


def _roofline_hbm(launch_bytes: float, per_launch_s: float, key: str, kernel: str, n_launch: int) -> dict:
    achieved = launch_bytes / per_launch_s / 1e9
    traffic = read_traffic(key)
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_over_algorithmic": round(traffic / launch_bytes, 4) if traffic else None,
            "kernel": kernel, "algorithmic_bytes_per_launch": round(launch_bytes),
            "avg_launch_us": round(per_launch_s * 1e6, 3), "launches_per_step": n_launch}


DEP_TEXT = {"all": "every input of layer l read after every KV head of layer l-1 has finished (a model's "
                   "dependency: each q head of layer l depends on every head of layer l-1)",
            "head": "layer l's inputs of KV head h read as soon as head h of layer l-1 has written them "
                    "(each KV head's layers chain on their own)"}


def run_decode(args, scheme: str, headline: bool, mode: str = "chain", dep: str = "all") -> dict:
    """The 36-layer, 32k-context chained decode step on the int8t64 (``t64``) or per-token
    symmetric (``tok``) cache; returns the result dict (the headline line when ``headline``).
    ``mode`` "chain": every layer in one launch (``ChainedStep``, ``nkv_decode_layers_*``), with
    the inter-layer dependency ``dep``; "layers": one fused launch per layer (``update_attend``,
    ``nkv_decode_step_*``), each launch after the one before."""
    import torch

    from nova_amd.chain import ChainedStep
    from nova_amd.kvattn import KVInt8Cache
    from nova_amd.kvtok import KVInt8TokCache

    dev = torch.device("cuda:0")
    L, ctx, W, K = args.layers, args.ctx, args.warmup, args.steps
    max_len = -(-(ctx + 3 * (W + K) + SETTLE_STEPS + 8) // 64) * 64
    cls = KVInt8TokCache if scheme == "tok" else KVInt8Cache
    cache = cls(num_slots=L, num_kv_heads=HKV, head_dim=D, max_len=max_len, num_q_heads=HQ, device=dev)
    if args.parts:
        cache.set_parts(args.parts)

    # ---- prefill: seeded N(0,1) K/V, 4 random K channels per head x8, quantized into the cache
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

    # ---- chained layers: layer l reads q / k / v from layer l-1's output buffer
    outs = (torch.randn(L, 1, HQ, 1, D, generator=gen, device=dev) / D ** 0.5).half()

    def layer_inputs(layer: int):
        prev = outs[layer - 1]  # layer 0: the previous step's last layer
        return prev[:, 0::HQ // HKV], prev[:, 1::HQ // HKV], prev

    chain = None
    if mode == "chain":
        ins = [layer_inputs(layer) for layer in range(L)]
        chain = ChainedStep(cache, [i[0] for i in ins], [i[1] for i in ins], [i[2] for i in ins],
                            [outs[layer] for layer in range(L)], n_parts=args.parts, dep=dep)

        def launches():
            chain()
    else:
        def launches():
            for layer in range(L):
                k, v, q = layer_inputs(layer)
                cache.update_attend(k, v, q, layer, out=outs[layer])

    def step():
        launches()
        cache.pos.add_(1)

    stream = torch.cuda.current_stream(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(SETTLE_STEPS + W):  # the clocks settle, then the W warmup steps
        graph.replay()
    torch.cuda.synchronize()
    pos0 = int(cache.pos.item())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    core_clk = core_clock(dev)
    ms = e0.elapsed_time(e1)
    assert int(cache.pos.item()) == pos0 + K
    if chain is not None:
        chain.check()  # no wait gave up (every workgroup was resident)
    assert torch.isfinite(outs).all()

    # ---- the launches alone (pos fixed): the chained launch, or the step's 36 chained launches
    g_launch = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_launch):
        launches()
    pos_l = int(cache.pos.item())
    ms_launches = _time_graph(g_launch, stream, K, W, SETTLE_STEPS)  # (pos fixed: settling moves nothing)
    if chain is not None:
        chain.check()
    # (the launches' graph: pos stays fixed, so every replay does the whole step's work; the step
    # graph would run past the cache's capacity during amd-smi's run and then attend nothing)
    clock = None if args.no_clock else clock_under_load(g_launch.replay)
    _calibration_copy(dev)

    ms_step = ms / K
    us = [pos0 + i + 1 for i in range(K)]  # tokens written when each timed step attends
    step_bytes = sum(step_launch_bytes(u, scheme) for u in us) / K * L
    n_launch = 1 if mode == "chain" else L
    launch_bytes = step_launch_bytes(pos_l + 1, scheme) * (L // n_launch)
    per_launch_s = ms_launches / 1e3 / n_launch
    kidx = 1 if scheme == "tok" else 0
    if mode == "chain":
        kname = (f"nkv::attn_layers_kernel<{kidx}> chained decode step ({L} layers x (append + split-K "
                 f"partials + merge), one launch per step, {cache_parts(chain)})")
    else:
        kname = (f"nkv::attn_prefix_kernel<{kidx}> fused decode step (append + split-K partials + "
                 "last-workgroup tail), one launch per layer")
    fmt = ("tok (int8 codes, one fp16 absmax scale per token and KV head)" if scheme == "tok"
           else "int8t64 (uint8 codes, fp16 min/step per 64 tokens per channel)")
    how = (f"all layers in one launch, {'all-head' if dep == 'all' else 'per-head'} dependency between layers"
           if mode == "chain" else "one launch per layer, each after the one before")
    res = {
        "metric": "int8-KV decode attention tokens/s + achieved HBM GB/s (% of peak) at 32k ctx",
        "value": round(K / (ms / 1e3), 2), "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic", "settle_steps": SETTLE_STEPS,
        "config": {"workload": f"{'per-token symmetric int8' if scheme == 'tok' else 'int8t64'} KV decode step, "
                               f"{L} layers x (32 q / 8 kv heads, head_dim 128), batch 1, {ctx}-token prefilled "
                               f"cache, layers chained through their outputs, {K} hipGraph-replayed steps, {how}",
                   "layers": L, "context": ctx, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "batch": 1,
                   "kv_format": fmt, "launch": mode,
                   "dependency": DEP_TEXT[dep] if mode == "chain" else "each layer's launch after the layer before",
                   "parts_per_head": chain.n_parts if mode == "chain" else cache._n_parts},
        "step_gbs": round(step_bytes / (ms_step / 1e3) / 1e9, 1),
        "step_pct_of_hbm_peak": round(100 * step_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
        "wall_s_timed": round(wall, 4),
        "roofline": _roofline_hbm(launch_bytes, per_launch_s, f"{mode}_{scheme}", kname, n_launch),
        "core_clock": core_clk,
        "gpu_clock": clock,
    }
    del graph, g_launch, cache, outs, chain
    torch.cuda.empty_cache()
    return res


def cache_parts(chain) -> str:
    return f"{chain.n_parts} streaming + 1 merging workgroups per KV head"


def run_paged(args, steps: int | None = None, scheme: str = "t64") -> dict:
    """Batched ragged decode: 8 sequences with seeded uniform lengths in [1024, 16384] (seed 3),
    36 layers, pages of 64 tokens (int8t64, or the per-token symmetric format with
    ``scheme="tok"``); one step = every layer's append + attention for all 8 sequences, captured
    as one hipGraph. Batch tokens/s; GB/s over the algorithmic bytes of the valid tokens (padding
    excluded)."""
    import torch

    from nova_amd.paged import PagedKVInt8Cache, PagedKVInt8TokCache

    dev = torch.device("cuda:0")
    L, B, W = args.layers, 8, args.warmup
    K = steps or 128
    lens = [int(x) for x in torch.randint(1024, 16385, (B,), generator=torch.Generator().manual_seed(3))]
    S = SETTLE_STEPS  # untimed step replays before the W warmup ones: the clocks settle, as for the decode
    per_seq = max(-(-(n + S + W + K + 2) // 64) for n in lens)
    total_pages = sum(-(-(n + S + W + K + 2) // 64) for n in lens)
    cls = PagedKVInt8TokCache if scheme == "tok" else PagedKVInt8Cache
    cache = cls(L, HKV, D, HQ, max_seqs=B, num_pages=total_pages, max_pages_per_seq=per_seq, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    for b, n in enumerate(lens):
        cache.reserve(b, n + S + W + K + 1)
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
    for _ in range(S + W):
        graph.replay()
    cache.note_advanced(S + W)
    torch.cuda.synchronize()
    ms = _time_graph(graph, stream, K, 0)
    cache.note_advanced(K)
    assert torch.isfinite(cache.merged[:B]).all()
    step_bytes = sum(sum(step_launch_bytes(n + S + W + i + 1, scheme) for n in lens) for i in range(K)) / K * L
    gbs = step_bytes / (ms / 1e3) / 1e9

    # ---- the step's launches alone (pos fixed; each is the layer's only launch): the prefix kernel
    # with its fused per-(sequence, KV head) tails, which also append the new token
    g_launch = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_launch):
        for layer in range(L):
            cache.decode_step(ks[layer], vs[layer], qs[layer], layer)
    per_launch_s = _time_graph(g_launch, stream, K, W, SETTLE_STEPS) / 1e3 / L
    pos = [n + S + W + K for n in lens]
    launch_bytes = sum(step_launch_bytes(p + 1, scheme) for p in pos)
    _calibration_copy(dev)
    kidx = 3 if scheme == "tok" else 2
    kname = (f"nkv::attn_prefix_kernel<{kidx}> paged decode step (append of the new token + attention) of the "
             f"{B} sequences with fused per-(sequence, KV head) tails, one launch per layer")
    res = {"metric": "paged ragged batch int8-KV decode: batch tokens/s + achieved HBM GB/s (% of peak)",
           "value": round(B / (ms / 1e3), 2), "unit": "tokens/s", "steps": K, "ms_per_step": round(ms, 4),
           "config": {"workload": f"paged {'per-token symmetric int8' if scheme == 'tok' else 'int8t64'} decode, "
                                  f"{B} ragged sequences (lengths {lens}), {L} layers x "
                                  "(32 q / 8 kv heads, head_dim 128), 64-token pages, hipGraph-replayed steps",
                      "lengths": lens, "layers": L, "page_tokens": 64, "work_units_per_head": cache.total_parts,
                      "launches_per_layer": 1},
           "step_gbs": round(gbs, 1), "step_pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
           "algorithmic_bytes_per_step": round(step_bytes), "settle_steps": S,
           "roofline": _roofline_hbm(launch_bytes, per_launch_s, f"paged_{scheme}", kname, L)}
    del graph, g_launch, cache
    torch.cuda.empty_cache()
    return res


def run_prefill(args, steps: int | None = None) -> dict:
    """Chunked prefill over int8 KV: a 512-token fp16 query chunk attending causally to a
    16384-token int8t64 cache plus itself, 32 q / 8 KV heads, head_dim 128 (seed 4). HIP events
    over K graph replays of its two launches; TFLOP/s and MFMA utilisation against the dense
    fp16 peak, GB/s."""
    import torch

    from nova_amd import _lib
    from nova_amd.kvattn import int8_prefill_attend, pack_int8_kv

    dev = torch.device("cuda:0")
    M, U = 512, 16384
    K, W = steps or 64, args.warmup
    g = torch.Generator(device=dev).manual_seed(4)
    k = torch.randn(1, HKV, U, D, generator=g, device=dev).half()
    v = torch.randn(1, HKV, U, D, generator=g, device=dev).half()
    packed = pack_int8_kv(k, v)
    del k, v
    q = torch.randn(1, HQ, M, D, generator=g, device=dev).half()
    kc = torch.randn(1, HKV, M, D, generator=g, device=dev).half()
    vc = torch.randn(1, HKV, M, D, generator=g, device=dev).half()
    out = torch.empty_like(q)
    lib = _lib.load()
    splits = args.splits or int(lib.nkv_prefill_default_splits(HKV, HQ, M, U))
    scratch = torch.empty(int(lib.nkv_prefill_workspace_bytes(HKV, HQ, M, splits)), dtype=torch.uint8, device=dev)
    int8_prefill_attend(q, kc, vc, *packed, used=U, out=out, scratch=scratch, splits=splits)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        int8_prefill_attend(q, kc, vc, *packed, used=U, out=out, scratch=scratch, splits=splits)
    # (every replay recomputes the same chunk, so the settle replays change nothing but the clocks)
    ms = _time_graph(graph, torch.cuda.current_stream(dev), K, W, SETTLE_STEPS)
    core_clk = core_clock(dev)
    assert torch.isfinite(out).all()
    _calibration_copy(dev)
    flop = 2 * 2 * D * HQ * (M * U + M * (M + 1) // 2)
    nbytes = U * 2176 + 2 * M * HQ * D * 2 + 2 * M * HKV * D * 2  # codes + rulers, q + out, chunk K/V
    tflops = flop / (ms / 1e3) / 1e12
    traffic = read_traffic("prefill")
    return {"metric": "chunked-prefill attention over int8 KV: chunks/s, TFLOP/s, MFMA utilisation, GB/s",
            "value": round(1e3 / ms, 2), "unit": "chunks/s", "steps": K, "ms_per_step": round(ms, 4),
            "config": {"workload": f"{M}-token fp16 chunk causally over a {U}-token int8t64 cache plus itself, "
                                   "32 q / 8 kv heads, head_dim 128", "chunk": M, "cache_tokens": U,
                       "splits": splits},
            "flop_per_step": flop,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_FP16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4), "traffic": traffic,
                         "traffic_over_algorithmic": round(traffic / nbytes, 4) if traffic else None,
                         "kernel": "nkv::prefill_chunk_kernel + nkv::prefill_combine_kernel (the chunk's two "
                                   "launches, timed together)",
                         "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(ms * 1e3, 3)},
            "gbs": round(nbytes / (ms / 1e3) / 1e9, 1), "settle_steps": SETTLE_STEPS, "core_clock": core_clk}


def run_read_ceiling(args, steps: int | None = None) -> dict:
    """The HBM read ceiling of the decode path's load pattern, over the bytes one 36-layer step
    streams (36 buffers of one layer's 32k-context algorithmic bytes, 2.6 GB in all, rotated so
    that nothing is served from the caches): ``nkv_read_bw_lds`` (8 KiB chunks by nontemporal
    LDS-DMA, two per wave in flight, 256 workgroups of 8 waves, as the decode kernels stream)
    over the whole 2.6 GB in one launch and as 36 launches of one layer's bytes, and
    ``nkv_read_bw`` (plain 16-byte register loads) over the whole. HIP events over K graph
    replays of each."""
    import torch

    from nova_amd import _lib

    dev = torch.device("cuda:0")
    K, W = steps or 16, args.warmup
    per_layer = -(-attn_bytes(CTX + 1) // 8192) * 8192
    L = LAYERS
    buf = torch.empty(per_layer * L, dtype=torch.uint8, device=dev)
    buf.random_(0, 256, generator=torch.Generator(device=dev).manual_seed(7))
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev)
    out = {}
    for name, launches in (("lds_dma_one_launch", [(0, per_layer * L, "nkv_read_bw_lds", 256)]),
                           ("lds_dma_per_layer_launches",
                            [(i * per_layer, per_layer, "nkv_read_bw_lds", 256) for i in range(L)]),
                           ("register_loads_one_launch", [(0, per_layer * L, "nkv_read_bw", 4096)])):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for off, n, fn, blocks in launches:
                _lib.call(fn, buf.data_ptr() + off, n, sink.data_ptr(), blocks, _lib.stream_ptr(dev))
        ms = _time_graph(g, s, K, W)
        out[name] = {"tb_per_s": round(per_layer * L / (ms / 1e3) / 1e12, 3), "ms": round(ms, 4),
                     "frac_of_peak": round(per_layer * L / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                     "launches": len(launches)}
        del g
    del buf, sink
    torch.cuda.empty_cache()
    best = out["lds_dma_one_launch"]["tb_per_s"]
    return {"metric": "HBM read ceiling of the decode path's load pattern (TB/s)", "value": best,
            "unit": "TB/s", "steps": K, "ms_per_step": out["lds_dma_one_launch"]["ms"],
            "config": {"workload": f"{L} x {per_layer} B read ({per_layer * L / 1e9:.2f} GB, one 36-layer 32k "
                                   "step's algorithmic bytes), rotating buffers", "bytes": per_layer * L},
            "probes": out}


def _standalone(res: dict, args) -> dict:
    """A workload's dict as its own contract line."""
    out = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
           "steps": res["steps"], "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic"}
    out.update({k: v for k, v in res.items() if k not in out})
    return out


# ---------------------------------------------------------------- end to end (random-weight decoder)


def bench_e2e(args, steps: int | None = None) -> dict:
    """End-to-end graph decode of the random-weight decoder with Qwen3-4B geometry (36 layers,
    hidden 2560, 32 q / 8 KV heads of 128, SwiGLU 9728, vocab 151936, fp16 weights) over the
    int8t64 cache: the prompt (``--ctx`` random ids) is prefilled in streamed chunks, then each
    step (embed, 36 x [attention block: RMSNorm + qkv projection, q/k norm + RoPE, int8 append +
    attention, in one launch (``--e2e-separate``: three); o_proj + residual, SwiGLU gate/up +
    RMSNorm, down + residual], final RMSNorm + lm_head, argmax, pos += 1) is one hipGraph replay."""
    import torch

    from nova_amd.decode import GraphDecoder
    from nova_amd.skeleton import SkeletonConfig, SkeletonForCausalLM

    dev = torch.device("cuda:0")
    L, ctx, W, K = args.layers, args.ctx, args.warmup, steps or args.steps
    cfg = SkeletonConfig(num_hidden_layers=L, vocab_size=VOCAB_QWEN3_4B)
    model = SkeletonForCausalLM(cfg, seed=5, device=dev, dtype=torch.float16).eval()
    fused = not getattr(args, "e2e_separate", False)
    model.use_decode_kernels(True, fused_qkv=fused)
    max_len = -(-(ctx + 4 + SETTLE_STEPS + W + K + 1) // 64) * 64
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
    for _ in range(SETTLE_STEPS + W):  # the clocks settle (as for the decode), then the W warmup steps
        dec.step()
    torch.cuda.synchronize()
    pos0 = int(dec.cache.pos.item())
    ms = _time_graph(dec.graph, torch.cuda.current_stream(dev), K, 0)
    assert int(dec.cache.pos.item()) == pos0 + K
    assert torch.isfinite(dec.logits).all()
    lay0 = model.model.layers[0]
    w_layer = sum(t.numel() * 2 for t in (lay0.w_qkv, lay0.attn.o_proj.weight, lay0.w_gate_up,
                                          lay0.mlp.down_proj.weight, lay0.norm, lay0.post_norm,
                                          lay0.attn.q_norm, lay0.attn.k_norm))
    w_head = model.lm_head.weight.numel() * 2 + 4 * cfg.hidden_size
    kv_step = sum(attn_bytes(pos0 + i + 1) + APPEND_BYTES for i in range(K)) / K * L
    step_bytes = L * w_layer + w_head + kv_step
    gbs = step_bytes / (ms / 1e3) / 1e9
    return {"metric": "end-to-end graph-decode tokens/s, 36-layer Qwen3-4B-geometry decoder (random weights) "
                      "over the int8 KV cache at 32k ctx",
            "value": round(1e3 / ms, 2), "unit": "tokens/s", "steps": K, "ms_per_step": round(ms, 4),
            "config": {"workload": f"greedy decode, {L} layers (hidden {cfg.hidden_size}, SwiGLU "
                                   f"{cfg.intermediate_size}), vocab {cfg.vocab_size}, int8t64 KV, {ctx}-token "
                                   f"prompt prefilled in {args.chunk}-token streamed chunks",
                       "layers": L, "context": ctx, "prefill_chunk": args.chunk,
                       "attention_block": ("one launch per layer (input RMSNorm + qkv projection, q/k norm + RoPE, "
                                           "append + attention)" if fused else
                                           "three launches per layer (qkv GEMV, q/k norm + RoPE, append + attention)")},
            "algorithmic_bytes_per_step": round(step_bytes), "step_gbs": round(gbs, 1),
            "step_pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2), "prefill_s": round(prefill_s, 3),
            "prefill_tokens_per_s": round(ctx / prefill_s, 1), "settle_steps": SETTLE_STEPS}


# ---------------------------------------------------------------- main


def main() -> int:
    args = parse_args()
    if args.traffic_from:
        write_traffic(*args.traffic_from, key=args.traffic_key)
        return 0
    if args.counters_from:
        if not args.counters_kernel or not args.counters_name or not args.stats_cmd:
            raise SystemExit("--counters-from needs --counters-kernel, --counters-name and --stats-cmd")
        write_counters(args.counters_from, args.counters_kernel, args.counters_name, args.stats_cmd)
        return 0
    if args.stats_from:
        if not args.stats_name or not args.stats_cmd:
            raise SystemExit("--stats-from needs --stats-name and --stats-cmd")
        write_stats(args.stats_from, args.stats_name, args.stats_cmd)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not run here (the decode attention shards by "
              "KV head across GPUs with no exchange; see the design notes)", file=sys.stderr)
        return 2

    import torch

    from nova_amd import _lib

    _lib.load()
    torch.cuda.set_device(0)
    steps = args.steps if args.steps != 256 else None
    if args.workload == "paged":
        res = _standalone(run_paged(args, steps, args.scheme), args)
    elif args.workload == "prefill":
        res = _standalone(run_prefill(args, steps), args)
    elif args.workload == "e2e":
        res = _standalone(bench_e2e(args), args)
    elif args.workload == "read":
        res = _standalone(run_read_ceiling(args, steps), args)
    else:
        res = run_decode(args, args.scheme, headline=True, mode=args.mode, dep=args.dep)
        if not args.no_cpu_baseline:
            res["cpu_baseline"] = cpu_baseline(args.cpu_seconds, args.scheme, args.ctx, args.layers)
        else:
            res["cpu_baseline"] = None
        if args.workload is None and not args.only:
            extra = {}
            for name, fn in (("head_dep_decode", lambda: run_decode(args, "t64", False, "chain", "head")),
                             ("layer_launch_decode", lambda: run_decode(args, "t64", False, "layers")),
                             ("tok_decode", lambda: run_decode(args, "tok", False, "chain", "all")),
                             ("tok_head_dep_decode", lambda: run_decode(args, "tok", False, "chain", "head")),
                             ("tok_layer_launch_decode", lambda: run_decode(args, "tok", False, "layers")),
                             ("paged_batch", lambda: run_paged(args)),
                             ("paged_batch_tok", lambda: run_paged(args, scheme="tok")),
                             ("chunked_prefill", lambda: run_prefill(args)),
                             ("read_ceiling", lambda: run_read_ceiling(args)),
                             ("e2e_decode", lambda: bench_e2e(args, args.e2e_steps))):
                try:
                    extra[name] = fn()
                except Exception as e:  # noqa: BLE001 - one extra workload failing must not hide the headline
                    extra[name] = {"error": f"{type(e).__name__}: {e}"[:400]}
            for name in ("head_dep_decode", "layer_launch_decode", "tok_decode", "tok_head_dep_decode",
                         "tok_layer_launch_decode"):
                if "error" not in extra[name]:
                    t = extra[name]
                    extra[name] = {k: t[k] for k in ("value", "unit", "ms_per_step", "step_gbs",
                                                     "step_pct_of_hbm_peak", "roofline", "config")}
            res["workloads"] = extra
            rc = extra["read_ceiling"]
            if "error" not in rc:
                # the headline's kernel against the read rate its own load pattern reaches
                res["roofline"]["frac_of_read_ceiling"] = round(
                    res["roofline"]["achieved"] / (rc["value"] * 1e3), 4)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
