"""Build ``nova_amd/libnova_kv.so`` from the HIP sources in ``nova_amd/csrc`` (gfx950).

    python -m nova_amd.build            # compile every source, link the library

hipcc cross-compiles for gfx950 without a GPU. Flags:
- ``-fhip-fp32-correctly-rounded-divide-sqrt``: the quantizer's fp32 divisions must be
  IEEE correctly rounded to reproduce the reference's codes bit for bit;
- ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 instructions
  are generated (they are avoided on this hardware pool);
- no fast-math flags anywhere.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libnova_kv.so"
SOURCES = ("nkv_quant.hip", "nkv_attn.hip", "nkv_gemv.hip")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build nova_amd)")


def _compile(src: str) -> Path:
    BUILD.mkdir(exist_ok=True)
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link ``libnova_kv.so`` (always rebuilds)."""
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size} bytes)")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
