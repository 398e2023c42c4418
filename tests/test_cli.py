"""The CLI surface (nimbus_sampler/cli.py) without a GPU: argument parsing and
the reference's bench-kernel inputs (main.rs:375-384), pinned at indices
computed here with Python integers."""
import subprocess
import sys

import numpy as np

from conftest import PKG


def test_cli_help_runs_without_gpu():
    r = subprocess.run([sys.executable, "-m", "nimbus_sampler", "--help"], cwd=PKG,
                       capture_output=True, text=True)
    assert r.returncode == 0 and "bench-kernel" in r.stdout and "bench-sampler" in r.stdout


def test_bench_kernel_inputs_follow_reference_formulas():
    from nimbus_sampler import cli
    x, w_f32, w_i8, w_i4 = cli.reference_kernel_inputs()
    assert x.shape == (768,) and w_f32.shape == (50257 * 768,) and w_i4.shape == (50257 * 384,)
    assert x[0] == np.float32(-1.0) and x[96] == np.float32(1.0) and x[97] == np.float32(-1.0)
    for i in (1, 2, 12345, 50257 * 768 - 1):
        h = i * 2654435761
        assert w_f32[i] == (np.float32(h % 2000) - np.float32(1000.0)) / np.float32(10000.0)
        assert w_i8[i] == h % 256
    assert w_i8[1] == 177 and w_f32[1] == np.float32(761.0) / np.float32(10000.0)
    assert w_i4[7] == (7 * 2654435761) % 256
