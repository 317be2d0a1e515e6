"""Builds libh3hip.so from csrc/*.hip with hipcc for gfx950, in-tree (the library sits beside this file).

Flags that carry meaning:
  -ffp-contract=off                          every rounding step is the one written (fmas only where called)
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE float32 division and square root (the row statistics and the
                                             quantizer's step are compared bit for bit)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                             no packed float32 instructions
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libh3hip.so")
ARCH = "gfx950"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if p and os.path.exists(p):
            return p
    raise RuntimeError("hipcc not found")


# Per-file flags. attention.hip: the MFMA accumulators in VGPRs. The compiler's own choice put part of the 16-bit
# kernel's in AGPRs (200 + 96 registers: one wavefront a SIMD); in VGPRs it takes 210 (two a SIMD) and runs the
# 16-bit form at 4096 tokens x 32 x 128 in 324 instead of 423 us. The int8 kernels are unchanged.
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: str, obj: str) -> None:
    cmd = [hipcc(), *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{r.stderr[-6000:]}")
    warn = [l for l in r.stderr.splitlines() if "warning" in l and "packed-fp32-ops" not in l]
    if warn:
        sys.stderr.write("\n".join(warn[:20]) + "\n")


def build(jobs: int = 8) -> str:
    """Compiles every csrc/*.hip and links libh3hip.so; returns its path."""
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_compile, s, o) for s, o in zip(srcs, objs)]:
            f.result()
    tmp = LIB + ".tmp"
    # rocBLAS: the plain float GEMMs of h3s_linear / h3s_linear_acc
    libs = ["-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run([hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp, *libs], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"linking libh3hip.so failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
