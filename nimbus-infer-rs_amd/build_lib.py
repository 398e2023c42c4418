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
    "-Wall", "-Wno-unused-function",
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
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
