"""The C++ host mirror (include/nimbus_sampler.hpp) runs the reference's
unit tests (src/sampler.rs:223-266) as a native binary built by build()."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_bin", "test_sampler")


def _run(mode):
    assert os.path.exists(BIN), "tests/cpp/_bin/test_sampler missing: run __graft_entry__.build() first"
    r = subprocess.run([BIN, mode], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout


def test_cpp_mirror_host_checks():
    _run("cpu")


@pytest.mark.gpu
def test_cpp_mirror_reference_unit_tests_on_gpu():
    _run("gpu")
