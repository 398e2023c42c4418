"""GPU parity of the long-row kernel (nis_sample_batch with V > 53245, no
top-k): greedy, top-p off and top-p of any nucleus size on rows streamed
once and read again from cache, against the CPU oracle.  Where the rows fit
the kernel's rules the test also checks that none was handed to the general
path."""
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
    print(f"[long] {label} B={x.shape[0]} V={V} T={T} p={p} ld={ld}", flush=True)
    rep = compare(run_gpu(sampler, x, V, params, seeds, ld=ld), run_oracle(x, V, params, seeds),
                  greedy=params.greedy())
    print(f"[long] {label} -> {rep}", flush=True)
    return rep


def test_c4_every_mode(sampler):
    # the Llama-3 vocabulary config (ties at the max on every tenth row):
    # greedy, top-p 0.9 and top-p off, all on the long-row kernel
    from nimbus_sampler import workloads
    w = workloads.WORKLOADS["c4"]
    x = w.make(64)
    for T, p in [(0.0, 1.0), (0.8, 0.9), (0.8, 1.0), (1.2, 0.99)]:
        rep = _check(sampler, x, w.V, T, p, list(range(64)), label=f"c4-T{T}-p{p}")
        if T > 0.0:
            assert rep["fast_rows"] == 64, rep


@pytest.mark.parametrize("V", [53246, 65537, 200003, 1 << 20])
def test_long_sizes_and_layouts(sampler, V):
    rnd = np.random.Generator(np.random.PCG64(V))
    B = 8
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    for ld_extra, T, p in [(0, 0.8, 0.9), (1, 1.0, 0.97), (3, 0.0, 1.0), (2, 1.1, 1.0)]:
        rep = _check(sampler, x, V, T, p, list(range(B)), ld=V + ld_extra,
                     label=f"V{V}-ld+{ld_extra}")
        if T > 0.0:
            assert rep["fast_rows"] == B, rep


def test_long_flat_and_peaked_rows(sampler):
    # near-flat rows (the cutoff bucket refined), and huge peaks over noise
    # (the cutoff inside the noise: neither side fits the lists)
    rnd = np.random.Generator(np.random.PCG64(21))
    B, V = 16, 128256
    flat = rnd.uniform(-0.5, 0.5, size=(B, V)).astype(np.float32)
    rep = _check(sampler, flat, V, 1.3, 0.99, list(range(B)), label="flat")
    assert rep["fast_rows"] == B, rep
    peak = rnd.standard_normal((B, V), dtype=np.float32)
    for r in range(B):
        pos = rnd.choice(V, size=int(rnd.integers(1, 6)), replace=False)
        peak[r, pos] += rnd.uniform(6.0, 11.0, size=pos.size).astype(np.float32)
    rep = _check(sampler, peak, V, 1.0, 0.95, list(range(B)), label="peaked")
    assert rep["fast_rows"] == B, rep


def test_long_masked_and_non_finite(sampler):
    # masked (-inf) vocabulary, a far spike (declined, general path), and
    # rows with NaN / +inf (declined: the general path's special cases)
    rnd = np.random.Generator(np.random.PCG64(22))
    B, V = 12, 100000
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    x[0:3, ::2] = -np.inf
    x[3:5, :20000] = -np.inf
    x[5, 77] = np.float32(200.0)
    x[6, :] = -np.inf
    x[7, 5] = np.inf
    for T, p in [(0.0, 1.0), (0.9, 0.9), (0.9, 1.0)]:
        _check(sampler, x[:6], V, T, p, list(range(6)), label=f"masked-T{T}-p{p}")
        # all -inf and +inf rows: the reference's special branches
        # (sampler.rs:192-208); tokens and RNG states exactly
        import nimbus_sampler as ns
        params = ns.SamplingParams(temperature=T, top_p=p)
        gpu = run_gpu(sampler, x[6:8], V, params, [6, 7])
        ref = run_oracle(x[6:8], V, params, [6, 7])
        assert np.array_equal(gpu[0], ref[0]), (T, p, gpu[0], ref[0])
        assert np.array_equal(gpu[2], ref[2])
