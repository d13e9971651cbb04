"""Builds libdashmi.so, the HIP library behind the C ABI (include/dashmi.h), for gfx950.

Every translation unit under csrc/ is compiled with hipcc to an object, in parallel, then linked
into ``dashmag_amd/libdashmi.so`` (in-tree, so that it travels with the repository to a GPU box).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libdashmi.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 instructions are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-lambda-capture",
]


# Per-source flags. The gated-delta-rule state passes are chains of dependent steps run by one
# wavefront per SIMD: with the products' accumulators in ordinary vector registers, the state's
# decay and conversions work on them in place instead of moving every value out of and back into
# the accumulator registers at each step.
# The attention kernels are scheduled with the strategy that keeps memory instructions together
# (measured at head width 256, one wavefront per SIMD: forward 288 -> 262 us, dK/dV 759 -> 723 us,
# dQ 359 -> 346 us on the reference's T = 6144 shape; the same at widths 64 and 128 within noise),
# but for the head width 256 dK/dV kernel, whose occupancy-driven iterative scheduling took it to
# 690 us.
EXTRA = {"gdr_chunk_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "attention_fwd.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
         "attention_mfma_bwd.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
         "attention_bwd_w4.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-maxocc"]}


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(os.path.basename(src), []), "-x", "hip", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj, r.stderr


def build(verbose=False, jobs=8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, srcs))
    if verbose:
        for _, err in results:
            err = "\n".join(l for l in err.splitlines() if "packed-fp32-ops" not in l)
            if err.strip():
                print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    # hipBLASLt for the log-probability's plain GEMMs (the logits and the gradient's products)
    rocm_lib = os.path.join(os.path.dirname(os.path.dirname(HIPCC)), "lib")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           f"-L{rocm_lib}", f"-Wl,-rpath,{rocm_lib}", "-lhipblaslt"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


HOST_CHECK_SRC = os.path.join(os.path.dirname(HERE), "tests", "host", "dm_host_check.cpp")
HOST_CHECK = os.path.splitext(HOST_CHECK_SRC)[0]


def build_host_check() -> str:
    """Compiles tests/host/dm_host_check.cpp, a caller that binds only include/dashmi.h and links
    libdashmi.so (no HIP headers), with the host compiler."""
    cxx = os.environ.get("CXX", "g++")
    inc = os.path.join(os.path.dirname(HERE), "include")
    cmd = [cxx, "-O2", "-std=c++17", "-Wall", f"-I{inc}", HOST_CHECK_SRC, f"-L{HERE}", "-ldashmi",
           "-Wl,-rpath,$ORIGIN/../../dashmag_amd", "-o", HOST_CHECK]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{cxx} failed on {HOST_CHECK_SRC}:\n{r.stderr}")
    return HOST_CHECK


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_host_check())
