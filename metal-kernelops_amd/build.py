"""Build libmko.so (the gfx950 HIP kernels behind the C ABI of include/mko.h).

Usage: ``python metal-kernelops_amd/build.py [--verbose]``.  Compiles every
``csrc/*.hip`` to an object in parallel with hipcc for gfx950, then links the
shared library into ``metal_kernelops/_lib/libmko.so`` (in-tree, so it travels
with the source tree to the GPU host).  Packed-FP32 instructions are disabled for
all device code.  After linking, the built code objects are checked (``isa_check.py``): the
DPP wait states of the Mamba-1 backward's inline assembly, and that no kernel rounds a product
to float16 in one step; a problem fails the build.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "metal_kernelops", "_lib")
LIB = os.path.join(LIBDIR, "libmko.so")
ARCH = "gfx950"
if HERE not in sys.path:
    sys.path.insert(0, HERE)

DEVICE_FLAGS = [
    "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-command-line-argument",
]


def _hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; install ROCm or put hipcc on PATH")
    return path


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src, verbose):
    obj = os.path.join(OBJDIR, os.path.basename(src)[:-4] + ".o")
    cmd = [_hipcc(), *DEVICE_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose=False, jobs=None):
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    # the inline-assembly DPP multiply-adds of the Mamba-1 backward rely on the schedule around
    # them; a build whose schedule breaks their wait states must not ship
    import isa_check
    n = isa_check.check_object(os.path.join(OBJDIR, "selscan.o"))
    if verbose:
        print(f"DPP wait states checked: {n} v_fmac_f32_dpp in selscan.o", flush=True)
    # one rounding of float16 results in every kernel: the SSD backward's cancelling sums
    # assume that all of its kernels round the same products alike
    for obj in objs:
        isa_check.check_f16_rounding(obj)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(verbose=args.verbose))
    sys.exit(0)
