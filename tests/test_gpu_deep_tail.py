"""GPU parity where the drawn tokens lie far below the row maximum.

One spike per row and every other logit 11-16 (scaled) nats below it, so the
tail holds a large share of the mass and many rows draw a token 16-24 octaves
below the maximum.  The mass 2^(t) of such a token must still match the
oracle's exp(w - max) (sampler.rs:201-205) within 1e-6 relative: the
probability of the drawn token and the kept mass are checked on every drawn
row, at T = 1 and T = 0.3, with top-p off and at 0.99.  The same rows with
top-k = V - 1 on rows longer than the register kernels hold run the general
path (its octave-relative masses), which every declined row also takes.
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


def deep_tail_rows(B, V, T, lo, hi, seed):
    """Spike at a random index; others at spike - T * U[lo, hi) (scaled nats)."""
    g = np.random.Generator(np.random.PCG64(seed))
    x = np.empty((B, V), dtype=np.float32)
    for r in range(B):
        spike = np.float32(g.uniform(-4.0, 12.0))
        d = g.uniform(lo, hi, size=V) * T
        x[r] = (np.float64(spike) - d).astype(np.float32)
        x[r, int(g.integers(0, V))] = spike
    return x


def tail_depth_octaves(x, tokens, T):
    """Octaves below the row max of each token (only rows where it was drawn)."""
    m = x.max(axis=1).astype(np.float64)
    t = x[np.arange(x.shape[0]), tokens].astype(np.float64)
    return (m - t) / max(float(np.float32(T)), 1e-6) * np.log2(np.e)


@pytest.mark.parametrize("V,T,top_p,lo,hi,B", [
    (50257, 1.0, 1.0, 11.0, 13.0, 96),
    (50257, 1.0, 0.99, 11.0, 13.0, 96),
    (50257, 0.3, 1.0, 11.0, 13.0, 96),
    (50257, 0.3, 0.99, 11.0, 16.0, 96),
    (128256, 1.0, 1.0, 13.5, 14.5, 96),   # ~20 octaves deep, V of the Llama-3 vocabulary
    (1 << 20, 1.0, 1.0, 15.5, 16.5, 128),  # 22-24 octaves deep at the largest V
])
def test_deep_tail_probabilities(sampler, V, T, top_p, lo, hi, B):
    import nimbus_sampler as ns
    x = deep_tail_rows(B, V, T, lo, hi, seed=V + int(100 * T) + int(100 * top_p))
    params = ns.SamplingParams(temperature=T, top_p=top_p)
    seeds = list(range(3000, 3000 + B))
    print(f"[deep-tail] B={B} V={V} T={T} p={top_p} depth [{lo},{hi}) nats", flush=True)
    gpu = run_gpu(sampler, x, V, params, seeds)
    ref = run_oracle(x, V, params, seeds)
    rep = compare(gpu, ref, greedy=False)
    depth = tail_depth_octaves(x, ref[0], T)
    drawn_deep = int((depth >= 16.0).sum())
    rep["rows_drawing_16_octaves_deep"] = drawn_deep
    rep["deepest_draw_octaves"] = float(depth.max())
    print(f"[deep-tail] -> {rep}", flush=True)
    # the workload must actually exercise the deep tail
    assert drawn_deep >= 4, rep


@pytest.mark.parametrize("V,T,top_p,lo,hi,B", [
    (60000, 0.3, 1.0, 11.0, 13.0, 96),
    (60000, 0.3, 0.99, 11.0, 16.0, 96),
    (128256, 1.0, 0.99, 13.5, 14.5, 96),
])
def test_deep_tail_probabilities_general_path(sampler, V, T, top_p, lo, hi, B):
    # top-k = V - 1 (sampler.rs:103-116) removes the row minimum only; the
    # rows run sample_rows_kernel (the general path), whose masses must meet
    # the same 1e-6 bar 16-24 octaves below the max
    import nimbus_sampler as ns
    x = deep_tail_rows(B, V, T, lo, hi, seed=7 * V + int(100 * T) + int(100 * top_p))
    params = ns.SamplingParams(temperature=T, top_p=top_p, top_k=V - 1)
    seeds = list(range(4000, 4000 + B))
    print(f"[deep-tail general] B={B} V={V} T={T} p={top_p} k={V - 1} depth [{lo},{hi}) nats",
          flush=True)
    gpu = run_gpu(sampler, x, V, params, seeds)
    ref = run_oracle(x, V, params, seeds)
    rep = compare(gpu, ref, greedy=False)
    assert (gpu[1]["kernel"] == 2).all(), gpu[1]["kernel"].tolist()
    depth = tail_depth_octaves(x, ref[0], T)
    drawn_deep = int((depth >= 16.0).sum())
    rep["rows_drawing_16_octaves_deep"] = drawn_deep
    rep["deepest_draw_octaves"] = float(depth.max())
    print(f"[deep-tail general] -> {rep}", flush=True)
    assert drawn_deep >= 4, rep


@pytest.mark.parametrize("T", [0.8, 0.6])
def test_far_heads_top_p_off_on_the_resident_kernel(sampler, T):
    # top-p off: a forced token (a logit of 100 among N(0, 3) logits, ~170
    # octaves above the rest) or a head of 2-300 logits near 50; every wave's
    # total is rescaled to the row max exactly in f64, so such rows stay on
    # the resident kernel however far below the max the other waves lie
    import nimbus_sampler as ns
    rnd = np.random.Generator(np.random.PCG64(int(T * 10) + 41))
    B, V = 32, 50257
    x = (rnd.standard_normal((B, V)) * 3.0).astype(np.float32)
    for r in range(B):
        if r % 2:
            x[r, int(rnd.integers(0, V))] = np.float32(100.0)
        else:
            n = int(rnd.integers(2, 301))
            x[r, rnd.choice(V, size=n, replace=False)] = (50.0 + rnd.uniform(-3.0, 3.0, size=n)).astype(np.float32)
    params = ns.SamplingParams(temperature=T, top_p=1.0)
    seeds = list(range(500, 500 + B))
    print(f"[far-heads] resident B={B} V={V} T={T}", flush=True)
    gpu = run_gpu(sampler, x, V, params, seeds)
    rep = compare(gpu, run_oracle(x, V, params, seeds), greedy=False)
    print(f"[far-heads] -> {rep}", flush=True)
    st = gpu[1]
    assert ((st["kernel"] == 1) & (st["reject"] == 0)).all(), (st["kernel"].tolist(), st["reject"].tolist())
