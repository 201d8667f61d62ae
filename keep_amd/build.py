"""Build the gfx950 HIP library ``keep_amd/libkeep_amd.so`` in-tree.

Each source is compiled separately (in parallel) with ``hipcc`` for gfx950 and
the objects are linked into one shared library with a C ABI
(``include/keep_amd.h``). Packed-FP32 instructions are disabled on the device
side (``-packed-fp32-ops``). The decode-layer sources have their leading
kernel arguments preloaded into SGPRs by the dispatcher
(``-amdgpu-kernarg-preload-count``; the compiler keeps a loading prologue for
firmware without the feature), so their first loads do not wait for a
kernel-argument fetch.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libkeep_amd.so"
OBJ = PKG / "_build"
ARCH = os.environ.get("KEEP_AMD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["abi.cpp", "matvec.hip", "moe.hip", "moe_i8.hip", "moe_tiles.hip", "router.hip", "plan.hip", "gemm_q8.hip", "rht.hip", "layer.hip", "block.hip", "encode.hip"]
FLAGS = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-command-line-argument"]
# sources whose kernels take their first-needed arguments as leading scalars (at most 14 dwords)
PRELOAD = {"moe_i8.hip", "layer.hip"}
PRELOAD_FLAGS = ["-mllvm", "-amdgpu-kernarg-preload-count=14"]


def _compile(src: str) -> Path:
    obj = OBJ / (src + ".o")
    cmd = [HIPCC, *FLAGS, *(PRELOAD_FLAGS if src in PRELOAD else []), "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    build()
