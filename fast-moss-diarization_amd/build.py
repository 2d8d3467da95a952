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


# Sources whose kernels copy global -> LDS through lds_copy16 (fmd_common.h):
# an asm block that writes M0 and then issues global_load_lds.  M0 is a
# register the compiler may otherwise use itself, so the device assembly of
# these files is checked after every build: M0 may appear only in that
# block's `s_mov_b32 m0, sN`, with the global_load_lds two lines below.
LDS_COPY_SOURCES = ["gemm.hip", "attn_prefill.hip", "encoder_kernels.hip"]


def _device_asm(src: str) -> str:
    cmd = [hipcc(), "-x", "hip", *HIPFLAGS, "--cuda-device-only", "-S", "-o", "-",
           str(CSRC / src)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"device assembly failed: {src}\n{proc.stderr[-4000:]}")
    return proc.stdout


def check_m0(asm: str, src: str) -> int:
    """Every instruction naming m0 is an lds_copy16 block's `s_mov_b32 m0, sN`
    followed by `s_nop 0` and global_load_lds.  Returns the blocks seen."""
    import re

    lines = [ln.split(";")[0].strip() for ln in asm.splitlines()]
    seen = 0
    for i, ln in enumerate(lines):
        if not re.search(r"\bm0\b", ln):
            continue
        ok = (re.fullmatch(r"s_mov_b32 m0, s\d+", ln) is not None and i + 2 < len(lines) and
              lines[i + 1] == "s_nop 0" and lines[i + 2].startswith("global_load_lds"))
        if not ok:
            raise RuntimeError(f"{src}: M0 used outside a direct-to-LDS copy: {ln!r}")
        seen += 1
    return seen


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
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        blocks = list(ex.map(lambda src: check_m0(_device_asm(src), src), LDS_COPY_SOURCES))
    if verbose:
        print(f"built {OUT} (M0 only in {sum(blocks)} direct-to-LDS copy blocks)")
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
