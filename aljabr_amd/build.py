"""Build recipe for libaljabr_rocm.so (gfx950 only).

Compiles every ``csrc/*.hip`` file with hipcc into ``_build/`` and links the C
ABI library next to this file. Run ``python -m aljabr_amd.build``; the round
driver calls it through ``__graft_entry__.build()``. Cross-compiles without a
GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libaljabr_rocm.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# Packed-FP32 instructions are disabled for all device code (the compiler must
# not form v_pk_{add,mul,fma}_f32); the host pass warns that it does not know
# the feature, which is harmless.
# Kernel-argument preload: the leading scalar arguments of a kernel (up to 14
# dwords on gfx950) arrive in SGPRs at wave launch instead of being read from
# the argument buffer; the compiler also emits the fallback that reads them.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm",
                "-amdgpu-kernarg-preload-count=14"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    noise = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


HOST_SRC = os.path.join(HERE, "host")
SPI_LIB = os.path.join(HERE, "libaljabr_rocm_spi.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
CXX = os.environ.get("CXX") or shutil.which("g++") or "g++"


def build_spi(verbose: bool = True) -> str:
    """The C++ Backend-SPI mirror (host/*.cpp) over the C ABI. It binds
    libaljabr_rocm.so with dlopen when a session opens, so it links no HIP."""
    srcs = sorted(glob.glob(os.path.join(HOST_SRC, "*.cpp")))
    tmp = SPI_LIB + ".tmp"
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", f"-I{INCLUDE}", *srcs, "-ldl",
           "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for the SPI mirror:\n{res.stderr}")
    if res.stderr.strip():
        sys.stderr.write(res.stderr)
    os.replace(tmp, SPI_LIB)
    if verbose:
        print(f"built {SPI_LIB}")
    return SPI_LIB


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    build_spi(verbose)
    return LIB


if __name__ == "__main__":
    build()
