"""GPU parity of the dense top-p kernel (nis_sample_batch with 0.95 <= top_p
< 1): one exact histogram of the whole row built in the stream, the cutoff
bucket refined up to 64^3 buckets per octave, and the smaller side of the
cutoff recomputed (or every float4 when neither side fits its lists).

Each case compares against the CPU oracle on the same seeded rows; where
the dense kernel must take the rows itself (they fit its rules), the test
also checks that no row was handed to the general path.
"""
import numpy as np
import pytest

from parity_util import compare, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    import nimbus_sampler as ns
    s = ns.Sampler(0)
    yield s
    s.close()


def _check(sampler, x, V, T, p, seeds, ld=None, label=""):
    import nimbus_sampler as ns
    params = ns.SamplingParams(temperature=T, top_p=p)
    print(f"[dense] {label} B={x.shape[0]} V={V} T={T} p={p} ld={ld}", flush=True)
    rep = compare(run_gpu(sampler, x, V, params, seeds, ld=ld), run_oracle(x, V, params, seeds),
                  greedy=False)
    print(f"[dense] {label} -> {rep}", flush=True)
    return rep


@pytest.mark.parametrize("p", [0.95, 0.99, 0.999])
def test_flat_rows_refine_the_cutoff_bucket(sampler, p):
    # near-flat logits put hundreds of tokens in each 1/64-octave bucket, so
    # the cutoff bucket is histogrammed again at 64^2 (and 64^3) per octave
    rnd = np.random.Generator(np.random.PCG64(int(p * 1000)))
    B, V = 64, 50257
    x = rnd.uniform(-0.5, 0.5, size=(B, V)).astype(np.float32)
    for T in (0.7, 1.3):
        rep = _check(sampler, x, V, T, p, list(range(B)), label=f"flat-p{p}-T{T}")
        assert rep["fast_rows"] == B, rep


def test_peaked_rows_recompute_every_float4(sampler):
    # a few huge peaks over N(0,1) noise: the cutoff sits inside the noise, so
    # neither side of it fits the lists and every float4 is recomputed
    rnd = np.random.Generator(np.random.PCG64(11))
    B, V = 48, 50257
    x = rnd.standard_normal((B, V), dtype=np.float32)
    for r in range(B):
        pos = rnd.choice(V, size=int(rnd.integers(1, 6)), replace=False)
        x[r, pos] += rnd.uniform(6.0, 11.0, size=pos.size).astype(np.float32)
    rep = _check(sampler, x, V, 1.0, 0.95, list(range(B)), label="peaked")
    assert rep["fast_rows"] == B, rep


def test_lattice_ties_across_refinement_levels(sampler):
    # values on a coarse lattice: tie groups of hundreds of equal logits; the
    # cutoff group cannot be split by finer buckets, so a row whose cutoff
    # group has more than 64 members leaves for the general path (parity
    # either way), and smaller groups are ranked by index across waves
    rnd = np.random.Generator(np.random.PCG64(12))
    B, V = 48, 30000
    x = (rnd.integers(-40, 41, size=(B, V)) / 16.0).astype(np.float32)
    _check(sampler, x, V, 1.0, 0.97, list(range(B)), label="lattice")
    y = (rnd.integers(-4000, 4001, size=(B, V)) / 1024.0).astype(np.float32)
    rep = _check(sampler, y, V, 0.9, 0.99, list(range(B)), label="fine-lattice")
    assert rep["fast_rows"] >= B // 2, rep


def test_masked_vocabulary_and_far_spikes(sampler):
    # -inf (masked) entries, a masked first chunk, and one spike far above the
    # rest (more than 64 octaves above some waves' first reference: the row
    # runs again with every first reference raised to 63 octaves below the
    # row max, and stays on the kernel)
    rnd = np.random.Generator(np.random.PCG64(13))
    B, V = 32, 40000
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    x[0:8, ::3] = -np.inf
    x[8:16, :3000] = -np.inf
    x[16:20, rnd.integers(0, V, size=4)] = np.float32(60.0)
    x[20:24, 5] = np.float32(150.0)
    rep = _check(sampler, x, V, 1.0, 0.96, list(range(B)), label="masked")
    assert rep["fast_rows"] == B, rep
    rep = _check(sampler, x, V, 0.5, 0.999, list(range(B)), label="masked-deep")
    assert rep["fast_rows"] == B, rep


@pytest.mark.parametrize("p", [0.95, 0.99])
def test_far_heads_stay_on_the_kernel(sampler, p):
    # a head of 2-300 logits 70-80 octaves above the rest (their spread puts
    # the cutoff inside the head), and rows whose masked waves hold nothing
    # while the rest lies ~100 octaves above 0: both run again with raised
    # first references; the lowest waves then fold wholly into their floors
    rnd = np.random.Generator(np.random.PCG64(int(p * 100) + 17))
    B, V = 32, 50257
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(1.5)
    for r in range(16):
        n = int(rnd.integers(2, 301))
        pos = rnd.choice(V, size=n, replace=False)
        x[r, pos] = (50.0 + rnd.uniform(-3.0, 3.0, size=n)).astype(np.float32)
    for r in range(16, B):
        n = int(rnd.integers(V // 4, 3 * V // 4))
        st = int(rnd.integers(0, V - n))
        x[r] += np.float32(40.0)
        x[r, st:st + n] = -np.inf
    rep = _check(sampler, x, V, 1.0, p, list(range(B)), label=f"far-heads-p{p}")
    assert rep["fast_rows"] == B, rep
    rep = _check(sampler, x, V, 0.6, p, list(range(100, 100 + B)), label=f"far-heads-p{p}-T0.6")
    assert rep["fast_rows"] == B, rep


@pytest.mark.parametrize("ld_extra", [0, 1, 2, 3])
def test_dense_layouts(sampler, ld_extra):
    # misaligned and padded rows, sizes with empty waves and partial chunks
    for V in (256, 777, 4099, 53245):
        rnd = np.random.Generator(np.random.PCG64(V + ld_extra))
        B = 24
        x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(1.5)
        rep = _check(sampler, x, V, 1.1, 0.97, list(range(B)), ld=V + ld_extra,
                     label=f"layout-V{V}-ld+{ld_extra}")
        assert rep["fast_rows"] == B, rep


def test_headline_shape_on_the_dense_kernel(sampler):
    # the headline distribution at top-p 0.95: the dense kernel's kept-side
    # listing (few kept) against the oracle
    from nimbus_sampler import workloads
    x = workloads.headline(64)
    rep = _check(sampler, x, 50257, 0.8, 0.95, list(range(64)), label="headline-p0.95")
    assert rep["fast_rows"] == 64, rep
