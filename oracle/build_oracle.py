"""Build the CPU oracle (test infrastructure only) into oracle/liboracle.so.

The oracle restates nimbus-infer-rs src/sampler.rs in plain C.  It is built
with gcc, IEEE f64 semantics: no fast-math and no FMA contraction, so the
arithmetic follows the reference's operation order.

The reference itself is Rust and this image has no rustc/cargo, so there is
no oracle/_ref build of it; the restatement is pinned by the reference's
own test vectors and independent checks instead.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    cmd = [
        "gcc", "-O2", "-std=c11", "-fPIC", "-shared",
        "-fno-fast-math", "-ffp-contract=off", "-fexcess-precision=standard",
        "-Wall", "-Wextra", "-Wno-unused-parameter",
        os.path.join(HERE, "sampler_oracle.c"),
        "-o", LIB + ".tmp", "-lm", "-lpthread",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
