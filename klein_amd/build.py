"""Builds the gfx950 sampler library in-tree: klein_amd/lib/libklein_sampler.so (the C ABI of
include/klein_sampler.h plus the C++ klein::Sampler of csrc/sampler.h)."""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libklein_sampler.so")
SOURCES = ["kls_kernels.hip", "kls_sort.hip", "kls_ppl.hip", "kls_noalloc.hip", "kls_state.hip", "kls_api.cpp", "sampler.cpp"]
ARCH = os.environ.get("KLS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    "-ffp-contract=off",                      # the reference rounds every f32/f64 operation separately
    "-fno-gpu-flush-denormals-to-zero",       # keep f32 subnormals (expf results down to 2^-149)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def build(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libklein_sampler.so")
    os.replace(tmp, LIB)
    return LIB



def build_dropin_check() -> str:
    """tests/cpp/dropin_check: a C++ program that uses klein::Sampler (csrc/sampler.h) through the library."""
    src = os.path.join(ROOT, "tests", "cpp", "dropin_check.cpp")
    exe = os.path.join(ROOT, "tests", "cpp", "dropin_check")
    cmd = [os.environ.get("CXX", "g++"), "-std=c++17", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           src, "-L", LIBDIR, "-lklein_sampler", "-Wl,-rpath,$ORIGIN/../../klein_amd/lib", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("building tests/cpp/dropin_check failed")
    return exe


if __name__ == "__main__":
    print(build(verbose=True))
