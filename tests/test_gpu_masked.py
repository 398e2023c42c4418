"""Masked vocabularies: rows with a share of their entries at -inf, scattered
at random (as grammar-constrained decoding leaves them) or as one contiguous
block, through the sparse (top-p 0.9), dense (top-p 0.97), resident (top-p
off, greedy) and long-row kernels.  Every row must match the oracle's
sample() (parity_util.compare), and stay on its row kernel: a wave whose
first chunks are masked takes its reference from its other chunks (dense,
resident), the dense kernel's -inf entries spread over the floor octave,
and a sparse wave whose sample missed its data lists again at the threshold
published meanwhile.  The one case left to the general path: a sparse row
whose unmasked part is only a wave or two (a 90 % block): whether a wave
there finds a higher threshold already published depends on the waves'
timing, so the count of such rows varies from run to run (a few here).
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


def _rows(kind, frac, B, V, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    x = (g.standard_normal((B, V)) * 3.0).astype(np.float32)
    for r in range(B):
        if kind == "random":
            x[r, g.random(V) < frac] = -np.inf
        else:
            n = int(frac * V)
            st = int(g.integers(0, V - n + 1))
            x[r, st:st + n] = -np.inf
    return x


@pytest.mark.parametrize("kind", ["random", "block"])
@pytest.mark.parametrize("frac", [0.1, 0.5, 0.9, 0.99, 0.999])
def test_masked_rows_stay_on_the_kernels(sampler, kind, frac):
    import nimbus_sampler as ns
    B, V = 64, 50257
    x = _rows(kind, frac, B, V, int(frac * 1000) + (kind == "block"))
    for T, p in ((0.8, 0.9), (0.8, 0.97), (0.8, 1.0), (0.0, 1.0)):
        params = ns.SamplingParams(temperature=T, top_p=p)
        print(f"[masked] {kind} {frac} T={T} p={p}", flush=True)
        gpu = run_gpu(sampler, x, V, params, list(range(B)))
        ref = run_oracle(x, V, params, list(range(B)))
        compare(gpu, ref, greedy=params.greedy())
        st = gpu[1]
        on = int(((st["kernel"] == 1) & (st["reject"] == 0)).sum())
        allowed = 4 if (kind == "block" and frac == 0.9 and p == 0.9) else 0
        assert on >= B - allowed, (kind, frac, T, p, st["kernel"].tolist(), st["reject"].tolist())


@pytest.mark.parametrize("kind", ["random", "block"])
def test_masked_long_rows(sampler, kind):
    # V = 128256 (single-read and long-row kernels): parity only
    import nimbus_sampler as ns
    B, V = 8, 128256
    for frac in (0.5, 0.99):
        x = _rows(kind, frac, B, V, 77 + int(frac * 100))
        for T, p in ((0.8, 0.9), (0.8, 0.97), (0.8, 1.0), (0.0, 1.0)):
            params = ns.SamplingParams(temperature=T, top_p=p)
            print(f"[masked long] {kind} {frac} T={T} p={p}", flush=True)
            gpu = run_gpu(sampler, x, V, params, list(range(B)))
            ref = run_oracle(x, V, params, list(range(B)))
            compare(gpu, ref, greedy=params.greedy())
