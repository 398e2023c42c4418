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


def test_generate_help_runs_without_gpu():
    r = subprocess.run([sys.executable, "-m", "nimbus_sampler", "generate", "--help"], cwd=PKG,
                       capture_output=True, text=True)
    assert r.returncode == 0 and "--max-new-tokens" in r.stdout and "--stream" in r.stdout


def _bench():
    import importlib.util
    import os
    from conftest import ROOT
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_worker_count_follows_threads_rs(monkeypatch):
    import os
    b = _bench()
    monkeypatch.setenv("NIMBUS_THREADS", "3")
    assert b.reference_worker_count() == 3
    for bad in ("0", "-2", "x", ""):
        monkeypatch.setenv("NIMBUS_THREADS", bad)
        assert b.reference_worker_count() == len(os.sched_getaffinity(0))
    monkeypatch.delenv("NIMBUS_THREADS")
    assert b.reference_worker_count() == len(os.sched_getaffinity(0))
    h = b.host_cpu()
    assert h["nproc"] >= 1


def test_bench_routing_constants_match_the_library():
    import os
    import re
    from conftest import PKG
    b = _bench()
    for fn, name, val in (("resident_path.h", "kRMaxV", b.RESIDENT_MAX_V),
                          ("sparse_path.h", "kSMaxV", b.SPARSE_MAX_V),
                          ("long_sparse_path.h", "kLSMaxV", b.LONG_SPARSE_MAX_V)):
        with open(os.path.join(PKG, "csrc", fn)) as f:
            line = re.search(name + r"\s*=.*//\s*(\d+)", f.read()).group(1)
        assert int(line) == val, name
    assert b.routed_kernel(50257, 0.8, 0, 0.9, 1.0) == "sample_rows_sparse_kernel"
    assert b.routed_kernel(50257, 0.0, 0, 0.9, 1.0).endswith("<greedy>")
    assert b.routed_kernel(50257, 1.0, 0, 1.0, 1.0).endswith("<all>")
    assert b.routed_kernel(50257, 0.7, 50, 1.0, 1.0) == "sample_rows_sparse_topk_kernel"
    assert b.routed_kernel(50257, 0.7, 50, 0.9, 1.3, history=True) == "sample_rows_kernel"
    assert b.routed_kernel(128256, 0.7, 50, 0.9, 1.0) == "sample_rows_kernel"
    # long rows: top-p below 0.95 is read once; 0.95 and up, top-p off and
    # greedy take the long-row kernel, and so do rows past 262141; a penalty
    # history on a long row takes the general kernel
    assert b.routed_kernel(128256, 0.8, 0, 0.9, 1.0) == "sample_rows_long_sparse_kernel"
    assert b.routed_kernel(128256, 0.8, 0, 0.97, 1.0) == "sample_rows_long_kernel<top-p>"
    assert b.routed_kernel(300000, 0.8, 0, 0.9, 1.0) == "sample_rows_long_kernel<top-p>"
    assert b.routed_kernel(128256, 0.8, 0, 0.9, 1.2, history=True) == "sample_rows_kernel"


def test_bench_refuses_more_than_one_gpu():
    from conftest import ROOT
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
