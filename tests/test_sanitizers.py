"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the host code,
run on the CPU (no GPU needed):

- the oracle (oracle/sampler_oracle.c) under a driver that sends random and
  special rows through every branch of sample() and the threads.rs batch
  driver (tests/sanitize/oracle_driver.c);
- the C ABI's host side (nimbus-infer-rs_amd/csrc/capi.hip, host code
  instrumented, device code built as usual) under a driver that checks the
  host RNG against the oracle and every argument check reachable without a
  device (tests/sanitize/capi_driver.cpp).

Each binary aborts on the first sanitizer report."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "sanitize", "_bin")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1")


def _run(cmd, **kw):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, **kw)
    assert r.returncode == 0, " ".join(cmd) + "\n" + r.stdout[-4000:]
    return r.stdout


def test_oracle_under_asan_ubsan():
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    os.makedirs(BIN, exist_ok=True)
    exe = os.path.join(BIN, "oracle_driver")
    _run(["gcc", "-O1", "-g", "-std=c11", "-ffp-contract=off", *SAN, "-I" + os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests", "sanitize", "oracle_driver.c"),
          os.path.join(ROOT, "oracle", "sampler_oracle.c"), "-o", exe, "-lm", "-lpthread"])
    out = _run([exe], env=ENV, timeout=300)
    assert "clean" in out


def test_capi_host_code_under_asan_ubsan():
    hipcc = "/opt/rocm/bin/hipcc"
    clang = "/opt/rocm/llvm/bin/clang"
    if not (os.path.exists(hipcc) and os.path.exists(clang)):
        pytest.skip("ROCm compilers not available")
    os.makedirs(BIN, exist_ok=True)
    lib = os.path.join(BIN, "libnis_asan.so")
    obj = os.path.join(BIN, "oracle_asan.o")
    exe = os.path.join(BIN, "capi_driver")
    # the oracle with the same (clang) sanitizer runtime as the library
    _run([clang, "-O1", "-g", "-std=c11", "-ffp-contract=off", *SAN, "-I" + os.path.join(ROOT, "oracle"),
          "-c", os.path.join(ROOT, "oracle", "sampler_oracle.c"), "-o", obj])
    # host code instrumented; each sanitizer flag applies to the host pass only
    host_san = []
    for f in ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all",
              "-fno-omit-frame-pointer"]:
        host_san += ["-Xarch_host", f]
    _run([hipcc, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-shared",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-w", *host_san,
          "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "nimbus-infer-rs_amd", "csrc"),
          os.path.join(ROOT, "nimbus-infer-rs_amd", "csrc", "capi.hip"), "-o", lib])
    _run([clang + "++", "-O1", "-g", "-std=c++17", *SAN, "-I" + os.path.join(ROOT, "include"),
          os.path.join(ROOT, "tests", "sanitize", "capi_driver.cpp"), obj, "-L" + BIN, "-lnis_asan",
          "-Wl,-rpath," + BIN, "-o", exe])
    out = _run([exe], env=ENV, timeout=300)
    assert "clean" in out
