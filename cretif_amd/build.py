"""Build libcretif.so (gfx950 HIP kernels + C ABI + C++ layer) in-tree.

    python -m cretif_amd.build            # compile everything
    python -m cretif_amd.build --asm DIR  # also write per-kernel gfx950 assembly to DIR

hipcc cross-compiles for gfx950 without a GPU, so this runs in any container
with ROCm.  Objects go to cretif_amd/_build/, the library to
cretif_amd/libcretif.so (both git-ignored; the .so travels with the tree).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcretif.so")
ARCH = "gfx950"

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + CSRC,
]
# Device code: gfx950 only; packed-FP32 VALU ops disabled (the compiler would
# otherwise pair independent fp32 FMAs into v_pk_fma_f32).
# Kernel arguments are preloaded into SGPRs (gfx950 feature), so a wave's first
# loads do not wait on scalar-memory round trips for its arguments.
DEVICE = ["--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mllvm", "-amdgpu-kernarg-preload-count=16"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("command failed:\n  %s\n%s%s" % (" ".join(cmd), r.stdout, r.stderr))
    return r


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if src.endswith(".hip"):
        cmd = [HIPCC, "-x", "hip"] + COMMON + DEVICE + ["-c", src, "-o", obj]
    else:
        cmd = [HIPCC] + COMMON + ["-D__HIP_PLATFORM_AMD__", "-c", src, "-o", obj]
    _run(cmd)
    return obj


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + sorted(glob.glob(os.path.join(CSRC, "*.cpp")))


def build(jobs: int | None = None, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs)
    os.replace(tmp, LIB)
    if verbose:
        print("built", os.path.relpath(LIB, ROOT), "from", len(srcs), "sources")
    return LIB


def dump_asm(outdir: str):
    """Write gfx950 assembly of each .hip file (for inspecting the code the compiler made)."""
    os.makedirs(outdir, exist_ok=True)
    for src in glob.glob(os.path.join(CSRC, "*.hip")):
        out = os.path.join(outdir, os.path.basename(src) + ".s")
        _run([HIPCC, "-x", "hip"] + COMMON + DEVICE + ["--cuda-device-only", "-S", src, "-o", out])
        print("asm", out)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", default=None)
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    build(a.j)
    if a.asm:
        dump_asm(a.asm)
    sys.exit(0)
