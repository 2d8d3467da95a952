"""Builds libfmd_dec.so (gfx950 HIP kernels + the C ABI) in this directory.

Usage: python build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OUT = HERE / "libfmd_dec.so"
OBJDIR = HERE / "_build"

SOURCES = [
    "gemv.hip",
    "gemm.hip",
    "rowops.hip",
    "attn_decode.hip",
    "attn_prefill.hip",
    "weights.hip",
    "encoder_kernels.hip",
    "fmd_dec.cpp",
    "encoder.cpp",
    "forward.cpp",
    "engine.cpp",
]

# Packed FP32 ops are disabled for all device code (the compiler would
# otherwise form v_pk_{add,mul,fma}_f32 from float2 arithmetic).
HIPFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    "-Wno-unused-value",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> Path:
    obj = OBJDIR / (Path(src).stem + ".o")
    cmd = [hipcc(), "-x", "hip", *HIPFLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{proc.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    OBJDIR.mkdir(exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{proc.stderr[-6000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    try:
        build(a.jobs, verbose=True)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
