"""GPU parity of top-k (src/sampler.rs:103-116, applied at 187) inside the
sparse kernel's top-k form (sample_rows_sparse_topk_kernel).

top_k_filter keeps every value at or above the k-th largest (ties with it
included, so possibly more than k), then top_p_filter runs on what is left.
The kernel finds the bucket of the k-th largest by counting down its exact
histograms, ranks that bucket's members only when they straddle the k-th,
and searches the top-p cutoff on the top-k mass, never below that bucket.
Every row must match the oracle's sample(); rows whose k-th largest lies
below the kernel's listed range are declined and recomputed by the general
path (kernel 2), with the same result.
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


def _check(sampler, x, V, seeds, label, on_kernel=True, ld=None, **kw):
    import nimbus_sampler as ns
    params = ns.SamplingParams(**kw)
    print(f"[top-k] {label} B={x.shape[0]} V={V} {kw} ld={ld}", flush=True)
    gpu = run_gpu(sampler, x, V, params, seeds, ld=ld)
    ref = run_oracle(x, V, params, seeds)
    rep = compare(gpu, ref, greedy=params.greedy())
    st = gpu[1]
    if on_kernel:
        assert (st["kernel"] == 1).all() and (st["reject"] == 0).all(), \
            (label, st["kernel"].tolist(), st["reject"].tolist())
    print(f"[top-k] {label} -> {rep}", flush=True)
    return gpu, ref, rep


@pytest.mark.parametrize("k", [1, 2, 40, 50, 200, 1000])
@pytest.mark.parametrize("p", [0.9, 0.97, 1.0])
def test_headline_rows(sampler, k, p):
    # the headline's logits (N(0, 3^2), T = 0.8) with top-k on top of top-p:
    # small k cuts inside the nucleus, k = 1000 lies beyond it (top-p decides)
    from nimbus_sampler import workloads
    B, V = 64, 50257
    x = workloads.headline(B)
    # (k = 1000 reaches about as deep as the kernel's listing threshold: rows
    # whose 1000th largest lies below it are declined, NIS_REJECT_WINDOW)
    gpu, ref, _ = _check(sampler, x, V, list(range(B)), f"headline k={k} p={p}",
                         on_kernel=k < 1000, temperature=0.8, top_p=p, top_k=k)
    st = gpu[1]
    assert ((st["kernel"] == 1) | (st["reject"] == 3)).all(), (st["kernel"], st["reject"])
    assert (st["kernel"] == 1).sum() >= B // 2
    kept = ref[1]["kept"]
    assert (kept <= k).all(), kept  # (no value ties in these rows)


@pytest.mark.parametrize("name,k", [("c3", 50), ("c3", 400), ("c2", 20), ("c1", 50)])
def test_config_rows(sampler, name, k):
    from nimbus_sampler import workloads
    w = workloads.WORKLOADS[name]
    B = min(w.B, 64)
    x = w.make(w.B)[:B]
    # (c3's nucleus is a few dozen tokens, so its listing threshold sits high:
    # some rows' 400th largest lies below it and they are declined)
    gpu, _, _ = _check(sampler, x, w.V, list(range(B)), f"{name} k={k}", on_kernel=k <= 200,
                       temperature=w.temperature, top_p=w.top_p, top_k=k)
    st = gpu[1]
    assert ((st["kernel"] == 1) | (st["reject"] == 3)).all(), (st["kernel"], st["reject"])
    assert (st["kernel"] == 1).sum() >= B // 2


@pytest.mark.parametrize("k", [1, 3, 7, 25, 64])
@pytest.mark.parametrize("lattice,T", [(8, 1.0), (256, 4.0)])
def test_value_ties_at_the_kth(sampler, k, lattice, T):
    # logits on a 1/8 lattice: value ties everywhere near the top, so the
    # k-th largest usually shares its value with neighbours (all of them are
    # kept) and its bucket (1/64 octave of x/T) is that tie group; on a 1/256
    # lattice at T = 4 a bucket spans about 11 lattice steps, so the k-th's
    # bucket holds distinct values on both sides of it
    rnd = np.random.Generator(np.random.PCG64(100 + k + lattice))
    B, V = 48, 50257
    x = (np.round(rnd.standard_normal((B, V)) * 3.0 * lattice) / lattice).astype(np.float32)
    # rows 0 mod 4: the max duplicated at three more indices (k = 1 keeps all four)
    for r in range(0, B, 4):
        m = x[r].max()
        x[r, rnd.choice(V, size=3, replace=False)] = m
    for p in (0.8, 1.0):
        _, ref, _ = _check(sampler, x, V, list(range(B)), f"ties 1/{lattice} k={k} p={p}",
                           temperature=T, top_p=p, top_k=k)
        if p == 1.0 and lattice == 8:
            assert (ref[1]["kept"] >= k).all()
            assert (ref[1]["kept"] > k).any(), "no row kept more than k (ties at the k-th)"


def test_kth_below_the_listed_range_falls_back(sampler):
    # k of half the vocabulary: the k-th largest lies far below the kernel's
    # listing threshold, so the row is declined (kernel 2, the general path)
    # with the same answer; k = V - 1 likewise
    from nimbus_sampler import workloads
    B, V = 16, 50257
    x = workloads.headline(B)
    for k in (V // 2, V - 1):
        gpu, _, _ = _check(sampler, x, V, list(range(B)), f"large k={k}", on_kernel=False,
                           temperature=0.8, top_p=0.9, top_k=k)
        st = gpu[1]
        assert ((st["kernel"] == 2) & (st["reject"] == 3)).all(), (st["kernel"], st["reject"])


def test_misaligned_rows_and_sizes(sampler):
    # (at V of a few thousand a wave holds one or two chunks; the sparse
    # kernel declines many such rows, with or without top-k, and the general
    # path answers them: parity only there)
    rnd = np.random.Generator(np.random.PCG64(5))
    for V, ld in ((50257, 50261), (53245, 53248), (16389, 16390), (4100, 4103), (256, 257),
                  (1000, 1000)):
        B = 24
        x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(3.0)
        k = min(30, V // 8)
        _check(sampler, x, V, list(range(B)), f"layout V={V} ld={ld}", ld=ld, on_kernel=V >= 16389,
               temperature=0.9, top_p=0.9, top_k=k)


def test_low_temperature_and_peaks(sampler):
    # T = 0.2 (the row spans about 100 octaves of x c, past the kernel's
    # histogram ring, so its rows are declined to the general path as plain
    # top-p rows at that temperature are), and rows with one dominant token
    # where top-k and top-p both keep a single element
    rnd = np.random.Generator(np.random.PCG64(9))
    B, V = 32, 50257
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    x[::2, rnd.integers(0, V)] += np.float32(30.0)
    # (top-p off with k = 5 on a peak row keeps noise ~29 octaves below the
    # peak: past the 16 octaves in which the kernel's kept masses are exact,
    # so those rows are declined, NIS_REJECT_WINDOW; the others stay)
    for T, p, k in ((0.2, 0.9, 10), (0.2, 1.0, 3), (1.5, 0.5, 100), (1.5, 1.0, 5)):
        gpu, _, _ = _check(sampler, x, V, list(range(B)), f"T={T} p={p} k={k}",
                           on_kernel=(T, p) == (1.5, 0.5), temperature=T, top_p=p, top_k=k)
        if (T, p) == (1.5, 1.0):
            st = gpu[1]
            assert (st["kernel"][1::2] == 1).all() and (st["reject"][::2] == 3).all()


def test_top_k_decode_steps_stay_on_the_kernel(sampler):
    # nis_decode_step with top-k (no penalty): every row-step runs the
    # sparse kernel's top-k form; tokens and histories follow the oracle loop
    import test_gpu_decode as td
    kernels = []
    diverged, n_done, n_started, _ = td._run(sampler, B=24, V=50257, steps=6, cap=8,
                                             params_kw=dict(temperature=0.8, top_p=0.9, top_k=40),
                                             seed=404, kernels=kernels, sigma=3.0)
    assert diverged <= 1 and n_started > 0
    k = np.concatenate([a for a, _ in kernels])
    r = np.concatenate([b for _, b in kernels])
    assert k.size > 0 and (k == 1).all() and (r == 0).all(), (np.unique(k), np.unique(r))
