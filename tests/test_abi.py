"""The C ABI library loads on a CPU-only host and exports exactly what include/nova_kv.h declares.

No kernel is launched here: only host-side functions (version, workspace sizing) and
argument validation that returns before any launch are called.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "nova_kv.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(nkv_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    from nova_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail("nova_amd/libnova_kv.so is not built (python -m nova_amd.build)")
    return _lib.load(require_gpu=False)


def test_header_declares_the_path():
    names = _declared()
    for must in ("nkv_quantize_int8", "nkv_dequantize_int8", "nkv_attn_decode_t64", "nkv_append_t64",
                 "nkv_decode_step_t64", "nkv_tail_attend", "nkv_ring_mask"):
        assert must in names


def test_every_declared_symbol_is_exported_and_bound(lib):
    from nova_amd import _lib

    names = _declared()
    for name in names:
        assert hasattr(lib, name), f"{name} declared in nova_kv.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == names


def test_abi_version_and_host_helpers(lib):
    from nova_amd import _lib

    assert lib.nkv_abi_version() == _lib.ABI_VERSION
    # at least 8 rulers per workgroup (one per wave) and at most 256 workgroups (one per
    # CU): 32K tokens = 512 rulers per head over 8 heads -> 32 parts
    assert lib.nkv_attn_default_parts(8, 512) == 32
    assert lib.nkv_attn_default_parts(8, 64) == 8
    assert lib.nkv_attn_default_parts(8, 1) == 1
    assert lib.nkv_attn_default_parts(2, 4096) == 128
    # one partial = [acc: 4 heads x 128][m: 4][l: 4] floats, 16-byte aligned, per KV head,
    # plus the fused tail's publication area: per head a counter and a flag per partial (ints,
    # in 256-byte blocks)
    per_part = 8 * (4 * 128 + 8) * 4
    sync = lambda hkv, parts: -(-(hkv * (1 + max(1, parts)) * 4) // 256) * 256  # noqa: E731
    assert lib.nkv_attn_workspace_bytes(8, 32, 64) == 64 * per_part + sync(8, 64) == 64 * per_part + 2304
    assert lib.nkv_attn_workspace_bytes(8, 32, 32) == 32 * per_part + 1280
    assert lib.nkv_attn_workspace_bytes(8, 32, 0) == per_part + sync(8, 1)
    assert lib.nkv_attn_workspace_bytes(128, 128, 1) == 128 * (128 + 4) * 4 + sync(128, 1)
    # per KV head: total_parts prefix partial slots and up to as many ring slots (one per sequence);
    # one counter per (unit, head) bound
    assert lib.nkv_paged_workspace_bytes(8, 32, 40) == 2 * 40 * per_part + 8 * 40 * 4


def test_only_one_hip_runtime_is_mapped(lib):
    """torch's libamdhip64 and the library's must be one and the same mapping."""
    maps = Path("/proc/self/maps").read_text().splitlines()
    paths = {ln.split()[-1] for ln in maps if "libamdhip64" in ln}
    assert len(paths) == 1, paths


def test_validation_errors_return_before_launch(lib):
    """Bad arguments come back as status codes with a message; nothing is launched."""
    from nova_amd import _lib

    rc = lib.nkv_quantize_int8(None, 7, 0, 1, 1, 128, 64, 1, None, 0, None, None, 0, None)
    assert rc == _lib.NKV_ERR_INVALID
    assert b"dtype" in lib.nkv_last_error()
    rc = lib.nkv_quantize_int8(None, 0, 0, 1, 1, 128, 64, 5, None, 0, None, None, 0, None)
    assert rc == _lib.NKV_ERR_INVALID and b"axis" in lib.nkv_last_error()
    # Q heads not divisible by KV heads, head_dim other than 128
    args = [None] * 7 + [30, 8, 128, 64, 64, 1, None, None, None, None, None, None, None, None, None, 1 << 20,
                         0, None]
    assert lib.nkv_attn_decode_t64(*args) == _lib.NKV_ERR_INVALID
    assert b"divisible" in lib.nkv_last_error()
    args[7], args[9] = 32, 64
    assert lib.nkv_attn_decode_t64(*args) == _lib.NKV_ERR_UNSUPPORTED
    assert b"head_dim" in lib.nkv_last_error()
    assert lib.nkv_copy_bytes(None, None, 15, None) == _lib.NKV_ERR_INVALID
    assert lib.nkv_clock_probe(None, 8, 100, None) == _lib.NKV_ERR_INVALID
    assert lib.nkv_clock_probe(ctypes.c_void_p(16), 0, 100, None) == _lib.NKV_ERR_INVALID
    assert lib.nkv_clock_probe(ctypes.c_void_p(16), 8, 0, None) == _lib.NKV_ERR_INVALID
    assert lib.nkv_ring_mask(None, None, None, 64, None, None) == _lib.NKV_ERR_INVALID
    # decode-step projections: sizes and layouts are checked before anything is launched
    # (the non-null pointers below are never dereferenced)
    fake = 1 << 20
    assert lib.nkv_gemv(None, None, 1e-6, None, 4, 64, None, None, None) == _lib.NKV_ERR_INVALID
    assert lib.nkv_gemv(fake, None, 1e-6, fake, 4, 100, None, fake, None) == _lib.NKV_ERR_INVALID
    assert b"multiple of 8" in lib.nkv_last_error()
    assert lib.nkv_gemv(fake, None, 1e-6, fake, 4, 16392, None, fake, None) == _lib.NKV_ERR_INVALID
    assert lib.nkv_gemv(fake + 2, None, 1e-6, fake, 4, 64, None, fake, None) == _lib.NKV_ERR_UNSUPPORTED
    assert lib.nkv_swiglu_gemv(fake, None, 1e-6, fake, 0, 64, fake, None) == _lib.NKV_ERR_INVALID
    # outputs that overlap the input vector, or a residual they are shifted against, are races
    w2, r3 = 1 << 21, 1 << 22
    assert lib.nkv_gemv(fake, None, 1e-6, w2, 4, 64, None, fake + 16, None) == _lib.NKV_ERR_INVALID
    assert b"overlaps x" in lib.nkv_last_error()
    assert lib.nkv_gemv(fake, None, 1e-6, w2, 4, 64, r3, r3 + 2, None) == _lib.NKV_ERR_INVALID
    assert b"residual" in lib.nkv_last_error()
    assert lib.nkv_swiglu_gemv(fake, None, 1e-6, w2, 8, 64, fake + 120, None) == _lib.NKV_ERR_INVALID
    assert b"overlaps x" in lib.nkv_last_error()
    assert lib.nkv_gemv(fake, None, 1e-6, w2, 1 << 31, 64, None, r3, None) == _lib.NKV_ERR_INVALID
    assert lib.nkv_qk_norm_rope(fake, 32, 8, 64, fake, fake, 1e-6, fake, fake, None) == _lib.NKV_ERR_UNSUPPORTED
    assert b"head_dim" in lib.nkv_last_error()
    # the decode step on the library's scratch array: 8 KV heads x 64 parts of 16 query
    # heads need 4.26 MB of partials, more than the array's 4 MiB
    step = [fake] * 3 + [128] + [fake] * 13 + [128, 8, 128, 1 << 16, fake, fake]
    assert lib.nkv_decode_step_static_t64(*step, 64, None) == _lib.NKV_ERR_UNSUPPORTED
    assert b"static scratch" in lib.nkv_last_error()
    assert lib.nkv_decode_step_static_t64(*step, -1, None) == _lib.NKV_ERR_INVALID


def test_product_path_refuses_to_run_without_gpu():
    import torch

    from nova_amd import _lib

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError, match="GPU"):
        _lib.load()


def test_ctypes_argument_counts_match_header():
    """Each declaration's parameter count equals its ctypes argtypes length."""
    from nova_amd import _lib

    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for m in re.finditer(r"\b(nkv_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        name, params = m.group(1), m.group(2).strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert len(_lib.SIGNATURES[name][1]) == n, name
    assert ctypes.sizeof(ctypes.c_void_p) == 8


def test_chained_step_sizes_and_checks(lib):
    """Workspace sizing of the chained decode step (one partial block per layer and the sync
    words) and its argument checks, which return before any device query or launch."""
    import numpy as np

    from nova_amd import _lib

    per_part = 8 * (4 * 128 + 8) * 4  # one partial of 4 query heads, per KV head
    # n layer counters, the exit ticket, the error word and the launch counter
    sync = lambda n: -(-((n + 3) * 4) // 256) * 256  # noqa: E731
    # one layer's output as tagged words (two fp16 values per 8 bytes), then its 32 issue flags in
    # 8 copies (one per group of polling workgroups)
    fwd = 32 * 128 // 2 * 8 + 8 * 32 * 4
    assert lib.nkv_layers_workspace_bytes(8, 32, 31, 36) == 36 * (31 * per_part + fwd) + sync(36)
    assert lib.nkv_layers_workspace_bytes(8, 32, 1, 1) == per_part + fwd + 256
    assert lib.nkv_layers_workspace_bytes(8, 30, 31, 36) == 0 and lib.nkv_layers_workspace_bytes(8, 32, 0, 4) == 0
    fake = 1 << 20
    table = np.full((2, 13), fake, dtype=np.int64)
    scalars = [fake] * 5
    args = lambda hq, tab, n=2: ([fake, tab.ctypes.data, n, 128] + scalars  # noqa: E731
                                 + [hq, 8, 128, 4096, fake, 1 << 24, 0, 0, None])
    assert lib.nkv_decode_layers_t64(*args(30, table)) == _lib.NKV_ERR_INVALID
    assert b"divisible" in lib.nkv_last_error()
    bad = table.copy()
    bad[1, 4] = 0  # layer 1's kmn
    assert lib.nkv_decode_layers_t64(*args(32, bad)) == _lib.NKV_ERR_INVALID
    assert b"layer 1" in lib.nkv_last_error()
    bad[1, 4] = fake + 8  # unaligned
    assert lib.nkv_decode_layers_t64(*args(32, bad)) == _lib.NKV_ERR_INVALID
    no_scalars = [fake, table.ctypes.data, 2, 128, fake, fake, None, fake, fake, 32, 8, 128, 4096, fake, 1 << 24, 0,
                  0, None]
    assert lib.nkv_decode_layers_t64(*no_scalars) == _lib.NKV_ERR_INVALID
    tok = np.full((2, 9), fake, dtype=np.int64)
    assert lib.nkv_decode_layers_tok(fake, tok.ctypes.data, 2, 128, fake, fake, 32, 8, 128, 100, fake, 1 << 24, 0,
                                     0, None) == _lib.NKV_ERR_INVALID
    assert b"multiple of 64" in lib.nkv_last_error()
    assert lib.nkv_decode_layers_t64(*(args(32, table)[:-2] + [5, None])) == _lib.NKV_ERR_INVALID
    assert b"NKV_DEP_ALL" in lib.nkv_last_error()


def _chain_table(L: int, q_of, kv_of, gap: int = 1 << 16, tok: bool = False):
    """A chained-step layer table of fake, aligned addresses: layer j's output at
    base + j * (32 x 128 fp16 + gap); q_of(l) / kv_of(l) give layer l's q and k_new addresses
    (v_new = k_new + 128 elements), the cache pointers lie far away."""
    import numpy as np

    base, out_bytes = 1 << 30, 32 * 128 * 2
    out = [base + j * (out_bytes + gap) for j in range(L)]
    cols = 9 if tok else 13
    t = np.full((L, cols), 1 << 40, dtype=np.int64)
    for l in range(L):
        t[l, 0] = q_of(out, l)
        t[l, 1] = kv_of(out, l)
        t[l, 2] = kv_of(out, l) + 256
        t[l, cols - 2] = out[l]
        t[l, cols - 1] = 0  # no lse
    return t


def test_chained_step_input_rules(lib):
    """The rows a chained layer may read from earlier outputs under each dependency mode
    (host-only check, fake addresses): head-local views chain per head; another head's rows of
    an earlier layer need its counter (always given); another head's rows of the previous step
    (a later layer's output) need NKV_DEP_ALL; the same layer's output of another head, and rows
    straddling two heads' rows, are refused."""
    from nova_amd import _lib

    L, HEAD, ALL, OK, BAD = 4, _lib.NKV_DEP_HEAD, _lib.NKV_DEP_ALL, _lib.NKV_OK, _lib.NKV_ERR_INVALID
    prev = lambda out, l: out[(l - 1) % L]  # noqa: E731
    cases = [
        # (q, k_new, kv_head_stride, rc with HEAD, rc with ALL)
        ("bench views", prev, lambda o, l: prev(o, l), 512, OK, OK),
        ("k from the next KV head's rows", prev, lambda o, l: prev(o, l) + 4 * 128 * 2, 512, BAD, OK),
        ("k straddling two heads' rows", prev, lambda o, l: prev(o, l) + 448 * 2, 512, BAD, BAD),
        ("k from the same layer's output, next head", prev, lambda o, l: o[l] + 4 * 128 * 2, 512, BAD, BAD),
        ("q and k in place, own head", lambda o, l: o[l], lambda o, l: o[l], 512, OK, OK),
        ("k from two layers back, next head", prev, lambda o, l: o[(l - 2) % L] + 4 * 128 * 2, 512, BAD, OK),
        ("inputs outside every output", lambda o, l: o[l] + 32 * 128 * 2, lambda o, l: o[l] + 32 * 128 * 2 + 4096,
         256, OK, OK),
    ]
    for name, q_of, kv_of, hs, want_head, want_all in cases:
        for tok in (False, True):
            t = _chain_table(L, q_of, kv_of, tok=tok)
            fn = lib.nkv_decode_layers_check_tok if tok else lib.nkv_decode_layers_check_t64
            for dep, want in ((HEAD, want_head), (ALL, want_all)):
                rc = fn(t.ctypes.data, L, hs, 32, 8, dep)
                assert rc == want, f"{name} (tok={tok}, dep={dep}): {rc} {lib.nkv_last_error()}"
    # layers 1.. read another head's rows of layer l - 1 (ordered by the counter), layer 0 reads
    # its own head's rows of the last layer: accepted in both modes
    kv = lambda o, l: prev(o, l) + (4 * 128 * 2 if l else 0)  # noqa: E731
    t = _chain_table(L, prev, kv)
    assert lib.nkv_decode_layers_check_t64(t.ctypes.data, L, 512, 32, 8, HEAD) == OK
    assert lib.nkv_decode_layers_check_t64(None, L, 512, 32, 8, HEAD) == BAD
    assert lib.nkv_decode_layers_check_t64(t.ctypes.data, L, 512, 32, 8, 2) == BAD
