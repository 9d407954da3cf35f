"""Build libdialq.so (the HIP kernels + C ABI) for gfx950, in-tree, and the
host operator layer above it (dial-27b_amd/host, C++ with a pybind11 module).

Usage: python dial-27b_amd/build.py [--jobs N]
Output: dial-27b_amd/lib/libdialq.so, dial-27b_amd/lib/dialq_host<ext-suffix>
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "lib")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(OUT, "libdialq.so")

SOURCES = ["abi.hip", "prep.hip", "gemv.hip", "gemm.hip", "local_q8.hip", "select.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # bit-defined float arithmetic: no contraction into FMA unless written
    "-ffp-contract=off",
    # no packed-FP32 VALU instructions (v_pk_fma_f32 & co.)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-I", os.path.join(HERE, "..", "include"),
]


# Per-source flags.  The decode GEMV's MFMAs write their accumulators to
# ordinary VGPRs: each tile's partial sums are read by VALU code right after
# the MFMAs, and the AGPR form added a v_accvgpr_read per value (8 per Q4_K
# tile); same occupancy, no spills, 27B layer decode +1.1-2.0 % (W8A16,
# FP8-128).  The prefill GEMMs keep the compiler's choice.
SOURCE_FLAGS = {"gemv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile {src} failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # the host pass does not know the packed-fp32 feature; that warning is harmless
    noise = [l for l in r.stderr.splitlines() if l.strip() and "packed-fp32-ops" not in l
             and "warning generated" not in l and "warnings generated" not in l]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def build(jobs: int = 0) -> str:
    os.makedirs(OUT, exist_ok=True)
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_host() -> str:
    """g++ build of host/dial_host.cpp, gguf.cpp, safetensors.cpp, sampling.cpp and bind.cpp into the pybind11
    module dialq_host, linked against libdialq.so, the HIP runtime and
    rocBLAS (RUNPATH: the library directory, then /opt/rocm/lib)."""
    import sysconfig
    import pybind11
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(OUT, "dialq_host" + suffix)
    host = os.path.join(HERE, "host")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(HERE, "..", "include"), "-I", "/opt/rocm/include",
           "-I", pybind11.get_include(), "-I", sysconfig.get_paths()["include"],
           os.path.join(host, "dial_host.cpp"), os.path.join(host, "gguf.cpp"), os.path.join(host, "safetensors.cpp"),
           os.path.join(host, "sampling.cpp"), os.path.join(host, "bind.cpp"),
           "-o", out + ".tmp", "-L", OUT, "-ldialq", "-L", "/opt/rocm/lib", "-lamdhip64", "-lrocblas",
           "-Wl,-rpath,$ORIGIN:/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host layer build failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=0)
    a = ap.parse_args()
    print(build(a.jobs))
    print(build_host())
