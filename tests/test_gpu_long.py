"""GPU parity of the long-row kernels (nis_sample_batch with V > 53245, no
top-k) against the CPU oracle: the single-read kernel for 0 < top-p < 0.95
(candidates listed in LDS against a pooled sampled threshold, the row read
once), and the long-row kernel for greedy, top-p off, top-p >= 0.95 and
penalty histories (the row read again from cache).  Where the rows fit a
kernel's rules the test also checks which method answered them
(nis_row_stats: kernel 1 with reject 0 for the single-read path, kernel 1
with the single-read path's reason for the long-row method behind it)."""
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
    # greedy, top-p 0.9 (read once), top-p off and 0.99 (the long-row kernel)
    from nimbus_sampler import workloads
    w = workloads.WORKLOADS["c4"]
    x = w.make(64)
    for T, p in [(0.0, 1.0), (0.8, 0.9), (0.8, 1.0), (1.2, 0.99)]:
        rep = _check(sampler, x, w.V, T, p, list(range(64)), label=f"c4-T{T}-p{p}")
        if T > 0.0:
            assert rep["fast_rows"] == 64, rep
        if p == 0.9:
            assert rep["sparse_rows"] == 64, rep  # every row answered by the single read


def test_c4_full_batch_single_read(sampler):
    # all 512 rows of the config stay on the single-read path (a declined row
    # would cost its CU two more reads of the row); parity on the first 64
    import nimbus_sampler as ns
    from nimbus_sampler import workloads
    w = workloads.WORKLOADS["c4"]
    x = w.make(512)
    params = ns.SamplingParams(temperature=0.8, top_p=0.9)
    gpu = run_gpu(sampler, x, w.V, params, list(range(512)))
    st = gpu[1]
    assert ((st["kernel"] == 1) & (st["reject"] == 0)).all(), (np.unique(st["kernel"]), np.unique(st["reject"]))
    sub = (gpu[0][:64], st[:64], gpu[2][:64])
    rep = compare(sub, run_oracle(x[:64], w.V, params, list(range(64))), greedy=False)
    print(f"[long] c4 B=512 -> {rep}", flush=True)


@pytest.mark.parametrize("V,ld_extra", [(53246, 0), (65537, 1), (100003, 3), (128256, 2), (151936, 0),
                                        (200003, 1), (262141, 0)])
def test_single_read_sizes_and_layouts(sampler, V, ld_extra):
    # N(0, 2^2) rows at T 0.8 (nucleus ~11% of the row at p 0.9): on the
    # single-read path while the lists hold that share (V up to ~160K),
    # declined to the long-row method past it; p 0.5 everywhere
    rnd = np.random.Generator(np.random.PCG64(V + 7))
    B = 8
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    for p in (0.9, 0.5):
        rep = _check(sampler, x, V, 0.8, p, list(range(B)), ld=V + ld_extra, label=f"single-read V{V} p{p}")
        assert rep["fast_rows"] == B, rep
        if V <= 151936 or p == 0.5:
            assert rep["sparse_rows"] == B, rep


def test_single_read_wide_nucleus_falls_back(sampler):
    # near-flat rows at p 0.9 keep ~90% of the row: far below the listing
    # threshold, so the single-read path declines (NIS_REJECT_WINDOW) and the
    # long-row method answers inside the same kernel
    import nimbus_sampler as ns
    rnd = np.random.Generator(np.random.PCG64(31))
    B, V = 8, 128256
    x = rnd.uniform(-0.5, 0.5, size=(B, V)).astype(np.float32)
    params = ns.SamplingParams(temperature=1.3, top_p=0.9)
    gpu = run_gpu(sampler, x, V, params, list(range(B)))
    st = gpu[1]
    assert ((st["kernel"] == 1) & (st["reject"] == 3)).all(), (st["kernel"], st["reject"])
    rep = compare(gpu, run_oracle(x, V, params, list(range(B))), greedy=False)
    print(f"[long] flat p0.9 -> {rep}", flush=True)


def test_single_read_peaks_low_temperature_and_ties(sampler):
    # (a) a spike 30-60 logits above N(0,1) noise: the sample's threshold lies
    # more than 31 octaves below the row max, so listed elements alias in the
    # histogram ring and are subtracted again; (b) T 0.1-0.3 on N(0, 3^2)
    # rows (the depth clamp); (c) values on a 1/64 lattice at T 1: each
    # lattice value holds hundreds of tied elements, more than either long
    # method ranks in its cutoff bucket, so these rows end on the general
    # path (parity only)
    rnd = np.random.Generator(np.random.PCG64(32))
    B, V = 12, 128256
    x = rnd.standard_normal((B, V), dtype=np.float32)
    for r in range(B):
        x[r, rnd.integers(0, V)] += np.float32(30.0 + 2.5 * r)
    rep = _check(sampler, x, V, 0.8, 0.9, list(range(B)), label="spikes")
    assert rep["sparse_rows"] == B, rep
    y = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(3.0)
    for T in (0.1, 0.2, 0.3):
        rep = _check(sampler, y, V, T, 0.9, list(range(B)), label=f"lowT{T}")
        assert rep["sparse_rows"] == B, rep
    z = (np.round(rnd.standard_normal((B, V)) * 2.0 * 64.0) / 64.0).astype(np.float32)
    for p in (0.9, 0.6):
        _check(sampler, z, V, 1.0, p, list(range(B)), label=f"lattice p{p}")


def test_single_read_crowded_cutoff_bucket(sampler):
    # a third of the row holds one value near the cutoff: its bucket has far
    # more members than one wave ranks, on the single-read path and on the
    # long-row method alike, so those rows end on the general path; the other
    # rows (100-250 members per cutoff bucket) stay on the single read
    import nimbus_sampler as ns
    rnd = np.random.Generator(np.random.PCG64(33))
    B, V = 6, 128256
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    x[:3, rnd.choice(V, size=V // 3, replace=False)] = np.float32(2.5)
    params = ns.SamplingParams(temperature=0.8, top_p=0.9)
    gpu = run_gpu(sampler, x, V, params, list(range(B)))
    rep = compare(gpu, run_oracle(x, V, params, list(range(B))), greedy=False)
    print(f"[long] crowded -> {rep} kernel={gpu[1]['kernel'].tolist()} reject={gpu[1]['reject'].tolist()}",
          flush=True)
    st = gpu[1]
    assert ((st["kernel"][3:] == 1) & (st["reject"][3:] == 0)).all(), (st["kernel"], st["reject"])


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


def test_long_far_heads_top_p_off(sampler):
    # top-p off at V = 128256: a forced token (a logit of 100 among N(0, 3)
    # logits) and rows with a masked half under logits near +40 at T = 0.6;
    # each wave's total is rescaled exactly in f64, so however far below the
    # max a wave lies the rows stay on the long-row kernel
    rnd = np.random.Generator(np.random.PCG64(61))
    B, V = 16, 128256
    x = (rnd.standard_normal((B, V)) * 3.0).astype(np.float32)
    for r in range(B):
        if r % 2:
            x[r, int(rnd.integers(0, V))] = np.float32(100.0)
        else:
            x[r] += np.float32(40.0)
            x[r, V // 4: 3 * V // 4] = -np.inf
    for T in (0.8, 0.6):
        rep = _check(sampler, x, V, T, 1.0, list(range(900, 900 + B)), label=f"far-heads-T{T}")
        assert rep["fast_rows"] == B, rep


@pytest.mark.parametrize("p", [0.95, 0.99])
def test_long_far_heads_top_p(sampler, p):
    # top-p >= 0.95 at V = 128256: a forced token (a logit of 100) or a
    # masked half under logits near +40 at T = 0.6 puts the row max 32 or
    # more octaves above some wave's first reference; the long-row launch
    # declines the row for that alone, and the pending launch runs the
    # long-row method again with every first reference raised to R - 31
    rnd = np.random.Generator(np.random.PCG64(int(p * 100) + 63))
    B, V = 16, 128256
    x = (rnd.standard_normal((B, V)) * 3.0).astype(np.float32)
    for r in range(B):
        if r % 2:
            x[r, int(rnd.integers(0, V))] = np.float32(100.0)
        else:
            x[r] += np.float32(40.0)
            x[r, V // 4: 3 * V // 4] = -np.inf
    for T in (0.8, 0.6):
        rep = _check(sampler, x, V, T, p, list(range(700, 700 + B)), label=f"far-heads-T{T}-p{p}")
        assert rep["fast_rows"] == B, rep


@pytest.mark.parametrize("V", [60000, 128256, 262080])
def test_long_greedy_with_penalty_histories(sampler, V):
    # greedy with a repetition-penalty history past 53245 (the long-row
    # kernel's greedy mode: the history as a bitmap in LDS, penalised values
    # compared in f64 beside the f32 max): histories holding each row's top
    # tokens at penalties above and below 1, ties between a penalised value
    # and a plain logit, rows of -inf with a history, misaligned rows
    import nimbus_sampler as ns
    from parity_util import compare, run_gpu, run_oracle
    rnd = np.random.Generator(np.random.PCG64(V + 5))
    B = 16
    x = (rnd.standard_normal((B, V)) * 3.0).astype(np.float32)
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [np.concatenate([order[r, : int(rnd.integers(1, 50))], rnd.integers(0, V + 10, size=60)])
           for r in range(B)]
    x[3, :] = -np.inf  # nothing exceeds work[0]: index 0
    x[4, 10] = np.float32(6.0)
    x[4, 20] = np.float32(3.0)  # penalised 6.0 / 2 == 3.0: the lower index wins
    gen[4] = np.array([10, 99], dtype=np.int64)
    off = np.zeros(B + 1, np.int64)
    off[1:] = np.cumsum([len(h) for h in gen])
    ids = np.concatenate(gen).astype(np.uint32)
    for pen in (2.0, 1.3, 0.5):
        params = ns.SamplingParams(temperature=0.0, repetition_penalty=pen)
        for ld in (V, V + 1):
            print(f"[long] greedy pen={pen} V={V} ld={ld}", flush=True)
            gpu = run_gpu(sampler, x, V, params, list(range(B)), ids, off, ld=ld)
            ref = run_oracle(x, V, params, list(range(B)), ids, off)
            compare(gpu, ref, greedy=True)
            st = gpu[1]
            assert ((st["kernel"] == 1) & (st["reject"] == 0)).all(), (st["kernel"].tolist(), st["reject"].tolist())


@pytest.mark.parametrize("V", [60000, 128256])
def test_long_top_p_off_with_penalty_histories(sampler, V):
    # top-p off with a repetition-penalty history past 53245 (the long-row
    # kernel's top-p-off mode: penalised values' masses 2^(y c - R_z) from
    # their f64 values, the max bound from them rounded up): histories of
    # each row's top tokens at penalties above and below 1, a row whose
    # penalised head rises far above the rest, misaligned rows
    import nimbus_sampler as ns
    from parity_util import compare, run_gpu, run_oracle
    rnd = np.random.Generator(np.random.PCG64(V + 9))
    B = 16
    x = (rnd.standard_normal((B, V)) * 3.0).astype(np.float32)
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [np.concatenate([order[r, : int(rnd.integers(1, 50))], rnd.integers(0, V + 10, size=60)])
           for r in range(B)]
    off = np.zeros(B + 1, np.int64)
    off[1:] = np.cumsum([len(h) for h in gen])
    ids = np.concatenate(gen).astype(np.uint32)
    for pen, T in ((1.3, 0.8), (2.0, 1.2), (0.5, 0.6)):
        params = ns.SamplingParams(temperature=T, top_p=1.0, repetition_penalty=pen)
        for ld in (V, V + 3):
            print(f"[long] top-p off pen={pen} T={T} V={V} ld={ld}", flush=True)
            seeds = list(range(40, 40 + B))
            gpu = run_gpu(sampler, x, V, params, seeds, ids, off, ld=ld)
            ref = run_oracle(x, V, params, seeds, ids, off)
            compare(gpu, ref, greedy=False)
            st = gpu[1]
            assert ((st["kernel"] == 1) & (st["reject"] == 0)).all(), (st["kernel"].tolist(), st["reject"].tolist())
