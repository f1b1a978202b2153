"""Builds libtinygiant_hip.so in-tree for gfx950 (hipcc), plus the
``libtinygiant.so`` alias that tinygiant/_lib.py's ``find_library`` looks for.

Usage: ``python -m tinygiant_amd.build`` (or ``__graft_entry__.build()``).
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtinygiant_hip.so"
ALIAS = PKG / "libtinygiant.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("TG_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # never let the backend form packed fp32 math
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
]
# per-source flags: the int8 MFMA expert phases take their MFMA results in
# VGPRs (no accumulator-register reads before the scale arithmetic)
HIP_EXTRA = {"tg_grouped_k.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HIP_SOURCES = ["tg_kernels.hip", "tg_grouped.hip", "tg_grouped_k.hip", "tg_decode.hip", "tg_decode_mx.hip", "tg_decode_rows.hip", "tg_head.hip", "tg_route.hip", "tg_attn.hip", "tg_api.hip"]
CXX_SOURCES = ["tg_host_ops.cpp"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}\n{r.stdout}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose=True):
    BUILD.mkdir(exist_ok=True)
    jobs = []
    objs = []
    for s in HIP_SOURCES:
        o = BUILD / (s + ".o")
        objs.append(o)
        jobs.append([HIPCC, *HIP_FLAGS, *HIP_EXTRA.get(s, []), "-I", str(CSRC), "-c", str(CSRC / s), "-o", str(o)])
    for s in CXX_SOURCES:
        o = BUILD / (s + ".o")
        objs.append(o)
        jobs.append(["g++", "-O2", "-fPIC", "-std=c++17", "-fvisibility=hidden", "-Wall", "-c", str(CSRC / s), "-o", str(o)])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        list(ex.map(_run, jobs))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if ALIAS.is_symlink() or ALIAS.exists():
        ALIAS.unlink()
    ALIAS.symlink_to(LIB.name)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
