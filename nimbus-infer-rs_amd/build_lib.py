"""Compile the gfx950 sampler library in-tree: lib/libnimbus_sampler.so.

hipcc builds the HIP kernels, the C ABI (include/nimbus_sampler.h) and the
C++ host mirror of the reference API into one shared library.  All HIP code
is compiled for gfx950 only, with packed-FP32 instruction selection
disabled.
"""
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libnimbus_sampler.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-bitwise-instead-of-logical",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]
SOURCES = ["capi.hip"]


def build(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    cmd = [HIPCC] + HIP_FLAGS + ["-shared"] + [os.path.join(CSRC, s) for s in SOURCES] + \
        ["-o", LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + out)
    if verbose and out.strip():
        print(out)
    os.replace(LIB + ".tmp", LIB)
    build_cpp_tests(verbose)
    return LIB


CPP_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_sampler.cpp")
CPP_TEST_BIN = os.path.join(ROOT, "tests", "cpp", "_bin", "test_sampler")


def build_cpp_tests(verbose: bool = False) -> str:
    """The C++ mirror of the reference's unit tests, linked against the
    library (rpath relative to the binary, so the tree can move)."""
    os.makedirs(os.path.dirname(CPP_TEST_BIN), exist_ok=True)
    rel = os.path.relpath(LIBDIR, os.path.dirname(CPP_TEST_BIN))
    cmd = [HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(ROOT, "include"), CPP_TEST_SRC,
           "-L" + LIBDIR, "-lnimbus_sampler", "-Wl,-rpath,$ORIGIN/" + rel,
           "-o", CPP_TEST_BIN + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc (C++ tests) failed:\n" + out)
    os.replace(CPP_TEST_BIN + ".tmp", CPP_TEST_BIN)
    return CPP_TEST_BIN


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
