"""CPU-side checks of the C ABI boundary (no GPU compute).

The HIP library must load, export every function include/nimbus_sampler.h
declares, agree with the header's struct layouts, and reject bad arguments
before touching a device.  Its host-side Rng functions are checked against
the RNG known answers.
"""
import ctypes
import json
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nimbus_sampler.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_0-9]+\s*\*?\s*(nis_\w+)\s*\(", text,
                                 re.M)))


def test_header_declares_expected_entry_points():
    import nimbus_sampler as ns
    assert set(declared_functions()) == set(ns.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    import nimbus_sampler as ns
    lib = ns.load_library()
    out = subprocess.run(["nm", "-D", "--defined-only", ns.LIB_PATH], check=True,
                         stdout=subprocess.PIPE, text=True).stdout
    exported = set(re.findall(r"\sT\s(nis_\w+)$", out, re.M))
    for name in declared_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None


def test_header_is_valid_c_with_expected_layouts(tmp_path):
    src = tmp_path / "abi_check.c"
    src.write_text(
        '#include "nimbus_sampler.h"\n'
        "#include <stddef.h>\n"
        "_Static_assert(sizeof(nis_params) == 24, \"nis_params\");\n"
        "_Static_assert(offsetof(nis_params, top_k) == 16, \"top_k\");\n"
        "_Static_assert(sizeof(nis_row_stats) == 64, \"nis_row_stats\");\n"
        "_Static_assert(offsetof(nis_row_stats, kept) == 40, \"kept\");\n"
        "_Static_assert(offsetof(nis_row_stats, path) == 48, \"path\");\n"
        "_Static_assert(sizeof(nis_weights) == 24, \"nis_weights\");\n"
        "_Static_assert(offsetof(nis_weights, d_data) == 8, \"d_data\");\n"
        "int main(void) { return 0; }\n")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only",
                    "-I" + os.path.join(ROOT, "include"), str(src)], check=True)
    import nimbus_sampler as ns
    assert ctypes.sizeof(ns.NisParams) == 24
    assert ns.ROW_STATS_DTYPE.itemsize == 64
    assert ns.ROW_STATS_DTYPE.fields["kept"][1] == 40
    assert ctypes.sizeof(ns.NisWeights) == 24 and ns.NisWeights.d_data.offset == 8


def test_host_rng_matches_kats():
    import nimbus_sampler as ns
    doc = json.load(open(os.path.join(ROOT, "tests", "golden", "rng_kats.json")))
    for k in doc["kats"]:
        r = ns.Rng(int(k["seed"]))
        assert r.state() == [int(v) for v in k["state"]]
        assert [r.next_u64() for _ in range(8)] == [int(v) for v in k["next_u64"]]
        assert ns.Rng(int(k["seed"])).next_f64() == float(k["first_f64"])
        r2 = ns.Rng.from_state([int(v) for v in k["state"]])
        assert r2.next_u64() == int(k["next_u64"][0])


def test_status_strings_and_null_context():
    import nimbus_sampler as ns
    L = ns.load_library()
    assert L.nis_status_string(ns.NIS_EINVAL) == b"invalid argument"
    assert L.nis_status_string(ns.NIS_ERANGE) == b"size out of range"
    assert L.nis_last_error(None) == b""
    p = ns.SamplingParams().to_c()
    assert L.nis_sample_batch(None, None, 1, 1, 1, ctypes.byref(p), None, None, None, None,
                              None) == ns.NIS_EINVAL
    assert L.nis_decode_step(None, None, 1, 1, 1, ctypes.byref(p), None, None, 1, None, None,
                             None, 0, None, None, None) == ns.NIS_EINVAL
    w = ns.NisWeights(ns.W_F32, 0, None, None)
    assert L.nis_lm_head_logits(None, None, 1, 1, 1, ctypes.byref(w), 1, None, 1) == ns.NIS_EINVAL
    assert L.nis_sync(None) == ns.NIS_EINVAL
    assert L.nis_ctx_create(0, None) == ns.NIS_EINVAL


def test_context_without_gpu_reports_nodev():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import nimbus_sampler as ns
    L = ns.load_library()
    ctx = ctypes.c_void_p()
    assert L.nis_ctx_create(0, ctypes.byref(ctx)) == ns.NIS_ENODEV
    with pytest.raises(ns.SamplerError):
        ns.Sampler(0)


def test_sampling_params_defaults_mirror_reference():
    import nimbus_sampler as ns
    p = ns.SamplingParams()   # sampler.rs:17-29
    assert (p.max_new_tokens, p.temperature, p.top_k, p.top_p, p.repetition_penalty, p.seed,
            p.stop_tokens) == (64, 1.0, 0, 1.0, 1.0, None, [])
    assert not p.greedy()
    assert ns.SamplingParams(temperature=0.0).greedy()
    assert ns.SamplingParams(temperature=-1.0).greedy()
    c = ns.SamplingParams(temperature=0.8, top_p=0.9).to_c()
    assert c.temperature == np.float32(0.8) and c.top_p == np.float32(0.9) and c.reserved == 0


def test_cpp_header_compiles_as_cpp17(tmp_path):
    """include/nimbus_sampler.hpp is self-contained C++17 over the C ABI."""
    import subprocess
    src = tmp_path / "t.cpp"
    src.write_text('#include "nimbus_sampler.hpp"\n'
                   'static_assert(sizeof(nis_params) == 24, "nis_params layout");\n'
                   'int main() { nimbus::SamplingParams p; return p.greedy() ? 1 : 0; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-fsyntax-only",
                        "-I" + os.path.join(ROOT, "include"), str(src)],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout
