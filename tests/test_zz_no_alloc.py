"""GPU test of nis_sample_one_noalloc, the allocation-free variant of
nis_sample_one that stages the row through a static device array: on the same
inputs it returns the same token and the same advanced RNG state as
nis_sample_one, call after call (the second call of each pair smaller, so
stale staging contents would show), and it rejects sizes beyond its limits."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_V = 1 << 18     # NIS_NOALLOC_MAX_V
MAX_GEN = 1 << 16   # NIS_NOALLOC_MAX_GEN


@pytest.fixture(scope="module")
def ctx():
    import nimbus_sampler as ns
    s = ns.Sampler(0)
    yield s
    s.close()


def _call(L, fn, ctx, x, params, gen, state):
    tok = ctypes.c_uint32(0xDEADBEEF)
    st = (ctypes.c_uint64 * 4)(*state)
    p = params.to_c()
    rc = getattr(L, fn)(ctx._ctx, ctypes.c_void_p(x.ctypes.data), x.size, ctypes.byref(p),
                        ctypes.c_void_p(gen.ctypes.data) if gen.size else None, gen.size, st,
                        ctypes.byref(tok))
    return rc, int(tok.value), [int(v) for v in st]


@pytest.mark.parametrize("sizes,kw", [
    ((50257, 4096), dict(temperature=0.8, top_p=0.9)),
    ((50257, 1000), dict(temperature=0.8, top_p=0.9, repetition_penalty=1.3)),
    ((MAX_V, 300), dict(temperature=1.0)),
    ((128256, 50257), dict(temperature=0.0)),
    ((4096, 7), dict(temperature=0.7, top_k=40, repetition_penalty=0.8)),
])
def test_noalloc_matches_sample_one(ctx, sizes, kw):
    import nimbus_sampler as ns
    L = ns.load_library()
    params = ns.SamplingParams(**kw)
    rnd = np.random.default_rng(sum(sizes))
    for call, V in enumerate(sizes):
        print(f"[noalloc] V={V} call={call} {kw}", flush=True)
        for row in range(3):
            x = (rnd.standard_normal(V) * 3.0).astype(np.float32)
            gen = rnd.integers(0, V, size=int(rnd.integers(0, 40)), dtype=np.uint32)
            state = ns.Rng(1000 * call + row).state()
            rc0, t0, s0 = _call(L, "nis_sample_one", ctx, x, params, gen, state)
            rc1, t1, s1 = _call(L, "nis_sample_one_noalloc", ctx, x, params, gen, state)
            assert rc0 == ns.NIS_OK and rc1 == ns.NIS_OK, (rc0, rc1)
            assert t1 == t0 and s1 == s0, (V, row, t0, t1)
            assert t1 < V


def test_noalloc_rejects_sizes_beyond_its_limits(ctx):
    import nimbus_sampler as ns
    L = ns.load_library()
    state = ns.Rng(1).state()
    big = np.zeros(MAX_V + 1, np.float32)
    rc, tok, st = _call(L, "nis_sample_one_noalloc", ctx, big, ns.SamplingParams(temperature=1.0),
                        np.zeros(0, np.uint32), state)
    assert rc == ns.NIS_ERANGE and tok == 0xDEADBEEF and st == state
    x = np.zeros(1000, np.float32)
    hist = np.zeros(MAX_GEN + 1, np.uint32)
    rc, _, _ = _call(L, "nis_sample_one_noalloc", ctx, x,
                     ns.SamplingParams(temperature=1.0, repetition_penalty=1.2), hist, state)
    assert rc == ns.NIS_ERANGE
    # without a penalty the history is not staged, so its length is not limited
    rc0, t0, s0 = _call(L, "nis_sample_one", ctx, x, ns.SamplingParams(temperature=1.0), hist, state)
    rc1, t1, s1 = _call(L, "nis_sample_one_noalloc", ctx, x, ns.SamplingParams(temperature=1.0),
                        hist, state)
    assert rc0 == rc1 == ns.NIS_OK and (t0, s0) == (t1, s1)
