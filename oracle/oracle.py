"""ctypes binding of the CPU oracle (oracle/sampler_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker / reported baseline and
never as the thing measured or shipped.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

# oracle_stats in sampler_oracle.h
STATS_DTYPE = np.dtype([
    ("max_w", "<f8"), ("z_kept", "<f8"), ("z_sorted", "<f8"), ("u", "<f8"),
    ("prob", "<f8"), ("topp_margin", "<f8"), ("cdf_margin", "<f8"),
    ("kept", "<u8"), ("path", "<u4"), ("token", "<u4"),
])
assert STATS_DTYPE.itemsize == 72

PATH_GREEDY, PATH_NONFINITE_MAX, PATH_BAD_TOTAL, PATH_DRAW, PATH_FALLTHROUGH = 1, 2, 3, 4, 5


class Params(ctypes.Structure):
    """oracle_params == nis_params layout (temperature, top_p, penalty, pad, top_k)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("_pad", ctypes.c_uint32),
                ("top_k", ctypes.c_uint64)]


def make_params(temperature=1.0, top_p=1.0, top_k=0, repetition_penalty=1.0):
    return Params(float(temperature), float(top_p), float(repetition_penalty), 0, int(top_k))


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        u64p = ctypes.POINTER(ctypes.c_uint64)
        L.oracle_rng_new.argtypes = [ctypes.c_uint64, u64p]
        L.oracle_rng_next_u64.argtypes = [u64p]
        L.oracle_rng_next_u64.restype = ctypes.c_uint64
        L.oracle_rng_next_f64.argtypes = [u64p]
        L.oracle_rng_next_f64.restype = ctypes.c_double
        dp = ctypes.POINTER(ctypes.c_double)
        L.oracle_apply_repetition_penalty.argtypes = [dp, ctypes.c_size_t, ctypes.c_void_p,
                                                      ctypes.c_size_t, ctypes.c_float]
        L.oracle_top_k_filter.argtypes = [dp, ctypes.c_size_t, ctypes.c_uint64]
        L.oracle_top_p_filter.argtypes = [dp, ctypes.c_size_t, ctypes.c_double, dp, dp]
        L.oracle_sample.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(Params),
                                    ctypes.c_void_p, ctypes.c_size_t, u64p, ctypes.c_void_p]
        L.oracle_sample.restype = ctypes.c_uint32
        L.oracle_sample_batch.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                          ctypes.c_int64, ctypes.POINTER(Params), ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_int]
        L.oracle_sample_batch.restype = ctypes.c_int
        _lib = L
    return _lib


class Rng:
    """Oracle Rng (sampler.rs:40-78) on a 4-word state."""

    def __init__(self, seed=None, state=None):
        self.state = (ctypes.c_uint64 * 4)()
        if state is not None:
            for i in range(4):
                self.state[i] = int(state[i])
        else:
            lib().oracle_rng_new(ctypes.c_uint64(int(seed) & (2**64 - 1)), self.state)

    def next_u64(self):
        return int(lib().oracle_rng_next_u64(self.state))

    def next_f64(self):
        return float(lib().oracle_rng_next_f64(self.state))

    def words(self):
        return [int(v) for v in self.state]


def rng_states(seeds):
    """[B,4] uint64 array of Rng::new(seed) states."""
    seeds = np.asarray(seeds, dtype=np.uint64).reshape(-1)
    out = np.zeros((seeds.size, 4), dtype=np.uint64)
    for i, s in enumerate(seeds):
        out[i] = Rng(int(s)).words()
    return out


def apply_repetition_penalty(logits_f64, generated, penalty):
    a = np.ascontiguousarray(logits_f64, dtype=np.float64).copy()
    g = np.ascontiguousarray(generated, dtype=np.uint32)
    lib().oracle_apply_repetition_penalty(a.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), a.size,
                                          g.ctypes.data if g.size else None, g.size,
                                          ctypes.c_float(penalty))
    return a


def top_k_filter(logits_f64, k):
    a = np.ascontiguousarray(logits_f64, dtype=np.float64).copy()
    lib().oracle_top_k_filter(a.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), a.size, int(k))
    return a


def top_p_filter(logits_f64, p):
    a = np.ascontiguousarray(logits_f64, dtype=np.float64).copy()
    margin = ctypes.c_double()
    ssum = ctypes.c_double()
    lib().oracle_top_p_filter(a.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), a.size,
                              ctypes.c_double(p), ctypes.byref(margin), ctypes.byref(ssum))
    return a, margin.value, ssum.value


def sample(logits_f32, params, generated=(), rng=None):
    """One sample() call; returns (token, stats record).  Advances `rng`."""
    x = np.ascontiguousarray(logits_f32, dtype=np.float32)
    g = np.ascontiguousarray(generated, dtype=np.uint32)
    st = np.zeros(1, dtype=STATS_DTYPE)
    tok = lib().oracle_sample(x.ctypes.data, x.size, ctypes.byref(params),
                              g.ctypes.data if g.size else None, g.size, rng.state,
                              st.ctypes.data)
    return int(tok), st[0]


def sample_batch(logits, V, params, states, gen_ids=None, gen_offsets=None, n_threads=0):
    """Batched oracle over rows of `logits` ([B, ld] float32, ld >= V).

    `states` ([B,4] uint64) is advanced in place.  Returns (tokens, stats,
    workers_used)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    B, ld = logits.shape
    assert states.dtype == np.uint64 and states.shape == (B, 4) and states.flags.c_contiguous
    tokens = np.zeros(B, dtype=np.uint32)
    stats = np.zeros(B, dtype=STATS_DTYPE)
    gi = go = None
    if gen_ids is not None:
        gen_ids = np.ascontiguousarray(gen_ids, dtype=np.uint32)
        gen_offsets = np.ascontiguousarray(gen_offsets, dtype=np.int64)
        gi, go = gen_ids.ctypes.data, gen_offsets.ctypes.data
    workers = lib().oracle_sample_batch(logits.ctypes.data, ld, B, V, ctypes.byref(params),
                                        states.ctypes.data, gi, go, tokens.ctypes.data,
                                        stats.ctypes.data, int(n_threads))
    return tokens, stats, workers
