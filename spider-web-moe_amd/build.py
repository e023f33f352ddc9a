"""Build libsmoe.so (the gfx950 HIP kernels + C ABI) in-tree.

    python spider-web-moe_amd/build.py [--jobs N]

Compiles every csrc/*.hip with hipcc for gfx950 and links
spider_moe_amd/lib/libsmoe.so.  No GPU is needed: hipcc cross-compiles.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "spider_moe_amd", "lib")
LIB = os.path.join(LIB_DIR, "libsmoe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-fvisibility=hidden",
    # code object v5: loadable by the HIP runtime that PyTorch-ROCm bundles
    # (libsmoe.so shares that runtime: it is loaded after torch and binds
    # to the already-loaded libamdhip64.so.7)
    "-mcode-object-version=5",
    # no packed-fp32 VALU ops in device code (hipcc's host pass warns that
    # it does not know the feature; that is harmless)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]


# Per-file additions.  smoe_front.hip: MFMA accumulators in VGPRs; left to
# choose, the compiler puts the logits kernel's 80 accumulators in AGPRs and
# rotates them with ~100 v_accvgpr moves per two K stages.
FILE_FLAGS = {
    "smoe_front.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(jobs: int = 4, verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    # the file name the reference's ctypes binding looks for
    # (kernels/python/spider_native.py:51-62): the host entry points of
    # include/spider_kernels.h live in the same library
    alias = os.path.join(LIB_DIR, "libspider_kernels.so")
    if os.path.lexists(alias):
        os.remove(alias)
    os.symlink(os.path.basename(LIB), alias)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    a = ap.parse_args()
    try:
        build(a.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
