"""Build libiian_pa.so (gfx950 HIP kernels + the C ABI of include/iian_pa.h) in-tree.

    python -m iian_amd.build

The library is written next to this file so that it travels with the source
tree; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libiian_pa.so"
SOURCES = ["pa_abi.hip", "pa_decode.hip", "pa_decode_q8.hip", "pa_prefill.hip", "pa_prefill16.hip", "pa_general.hip",
           "pa_kv_write.hip", "pa_batch.hip", "pa_rope.hip", "pa_runtime.hip"]
ARCH = "gfx950"

# Packed-FP32 VALU ops are disabled for all device code: some of their forms
# have given wrong results on these boxes.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libiian_pa.so")


def _compile(cc: str, src: str, objdir: Path, verbose: bool) -> str:
    obj = objdir / (Path(src).stem + ".o")
    cmd = [cc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    return str(obj)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 (in parallel) and link libiian_pa.so; returns its path."""
    cc = hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    jobs = max(1, min(len(SOURCES), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda src: _compile(cc, src, objdir, verbose), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libiian_pa.so failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
