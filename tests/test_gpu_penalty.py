"""GPU parity of the repetition penalty inside the register-resident kernels.

A top-p launch with a penalty history runs sample_rows_sparse_pen_kernel
(top-p < 0.95) or sample_rows_dense_pen_kernel (0.95 <= top-p < 1), which
apply apply_repetition_penalty (src/sampler.rs:83-101) in f64 to the row they
hold in registers.  The sparse kernel moves penalised logits to a side list
as the chunk lands; the dense kernel keeps them in registers and gives the
flagged chunks an f64 form of each step.  Greedy and top-p-off launches run
the resident kernel's penalised modes.  Every row must match the oracle's
sample() and stay on its kernel (stats kernel == 1, reject == 0): none may
fall back to the general path.
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


def _params(**kw):
    import nimbus_sampler as ns
    return ns.SamplingParams(**kw)


def _csr(gen):
    off = np.zeros(len(gen) + 1, np.int64)
    off[1:] = np.cumsum([len(g) for g in gen])
    ids = np.concatenate([np.asarray(g, np.int64) for g in gen]).astype(np.uint32) \
        if off[-1] else np.zeros(0, np.uint32)
    return ids, off


def _check(sampler, x, V, params, gen, label, on_kernel=True):
    ids, off = _csr(gen)
    seeds = list(range(x.shape[0]))
    print(f"[penalty] {label} B={x.shape[0]} V={V} T={params.temperature} p={params.top_p} "
          f"pen={params.repetition_penalty} n_ids={len(ids)}", flush=True)
    gpu = run_gpu(sampler, x, V, params, seeds, ids, off)
    ref = run_oracle(x, V, params, seeds, ids, off)
    rep = compare(gpu, ref, greedy=params.greedy())
    st = gpu[1]
    if on_kernel:
        assert (st["kernel"] == 1).all() and (st["reject"] == 0).all(), \
            (label, st["kernel"].tolist(), st["reject"].tolist())
    print(f"[penalty] {label} -> {rep}", flush=True)
    return gpu, ref


@pytest.mark.parametrize("pen", [1.3, 0.8, 2.0])
def test_random_histories(sampler, pen):
    # histories of 0..300 ids with repeats, some past V (ignored by the reference)
    from nimbus_sampler import workloads
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(int(pen * 100)))
    x = workloads.headline(B)
    gen = []
    for r in range(B):
        n = int(rnd.integers(0, 301))
        g = rnd.integers(0, V + 8, size=n)
        if n > 4:
            g[: n // 4] = g[n // 4: 2 * (n // 4)]  # repeats
        gen.append(g)
    _check(sampler, x, V, _params(temperature=0.8, top_p=0.9, repetition_penalty=pen), gen,
           f"random pen={pen}")


@pytest.mark.parametrize("pen,T", [(1.01, 0.8), (1.3, 0.8), (0.9, 1.0), (1.3, 0.5)])
def test_histories_on_the_nucleus(sampler, pen, T):
    # the history holds each row's top tokens, so penalised logits are kept,
    # ranked at the cutoff and drawn
    from nimbus_sampler import workloads
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(7 + int(pen * 100)))
    x = workloads.headline(B)
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [order[r, : int(rnd.integers(1, 120))] for r in range(B)]
    # a strong penalty on a row's whole head spreads its nucleus over
    # thousands of tokens, past what the sparse path lists: such rows are
    # declined and recomputed by the general path (checked for parity alike)
    gpu, _ = _check(sampler, x, V, _params(temperature=T, top_p=0.9, repetition_penalty=pen), gen,
                    f"nucleus pen={pen} T={T}", on_kernel=pen == 1.01)
    st = gpu[1]
    on = (st["kernel"] == 1) & (st["reject"] == 0)
    drew = sum(int(gpu[0][r]) in set(gen[r].tolist()) for r in np.nonzero(on)[0])
    print(f"[penalty] rows on the sparse kernel {int(on.sum())}/{B}, of which drew a penalised "
          f"token: {drew}", flush=True)
    if pen == 1.01:
        assert drew > B // 4


def test_ties_between_penalised_and_plain_values(sampler):
    # logits on a 1/16 lattice; penalty 2 maps a penalised 2v (or v/2 for
    # v <= 0) to exactly v, so penalised and plain elements tie in f64 and the
    # stable order (value, then index) decides at the cutoff
    B, V = 48, 50257
    rnd = np.random.Generator(np.random.PCG64(11))
    base = np.round(rnd.standard_normal((B, V)) * 48.0).astype(np.float32) / np.float32(16.0)
    gen = []
    for r in range(B):
        top = np.argsort(-base[r], kind="stable")[:400]
        idx = rnd.choice(top, size=int(rnd.integers(20, 200)), replace=False)
        pos = base[r, idx] > 0
        base[r, idx[pos]] *= np.float32(2.0)
        base[r, idx[~pos]] *= np.float32(0.5)
        gen.append(idx)
    for p in (0.5, 0.9):
        gpu, _ = _check(sampler, base, V, _params(temperature=0.8, top_p=p, repetition_penalty=2.0),
                        gen, f"ties p={p}", on_kernel=False)
        st = gpu[1]
        assert ((st["kernel"] == 1) & (st["reject"] == 0)).sum() >= 0.9 * B, \
            (st["kernel"].tolist(), st["reject"].tolist())


def test_padded_rows_and_short_vocabularies(sampler):
    # misaligned rows (ld not a multiple of 4) put penalised ids in the partial
    # head and tail slots; V at the small end of the kernel's range
    from nimbus_sampler import workloads
    rnd = np.random.Generator(np.random.PCG64(5))
    for V, ld in ((50257, 50261), (256, 259), (1000, 1000)):
        B = 16
        x = workloads.headline(B, V)
        gen = [np.concatenate([[0, 1, 2, V - 1, V - 2, V - 3],
                               rnd.integers(0, V, size=int(rnd.integers(0, 40)))])
               for _ in range(B)]
        ids, off = _csr(gen)
        params = _params(temperature=0.8, top_p=0.9, repetition_penalty=1.4)
        gpu = run_gpu(sampler, x, V, params, list(range(B)), ids, off, ld=ld)
        ref = run_oracle(x, V, params, list(range(B)), ids, off)
        compare(gpu, ref, greedy=False)
        if V == 50257:
            assert (gpu[1]["kernel"] == 1).all() and (gpu[1]["reject"] == 0).all(), (V, ld)


def test_crowded_histories_finish_on_the_dense_path(sampler):
    # more penalised elements in one wave's range than the sparse path's side
    # lists hold: the sparse launch marks those rows pending before anything
    # is written, and the pending launch finishes them on the dense path (up
    # to 16 penalised elements per lane); past that, on the general path
    from nimbus_sampler import workloads
    B, V = 9, 50257
    x = workloads.headline(B)
    gen = []
    for r in range(B):
        if r % 3 == 0:
            gen.append(np.arange(40000, 40010))        # short: the sparse path
        elif r % 3 == 1:
            gen.append(np.arange(0, 3000, 7))          # crowded: the dense path
        else:
            gen.append(np.arange(0, 4000))             # every element of a lane: general
    gpu, _ = _check(sampler, x, V, _params(temperature=0.8, top_p=0.9, repetition_penalty=1.3),
                    gen, "crowded", on_kernel=False)
    st = gpu[1]
    assert (st["kernel"][0::3] == 1).all() and (st["reject"][0::3] == 0).all()
    assert (st["kernel"][1::3] == 1).all() and (st["reject"][1::3] == 0).all()
    assert (st["kernel"][2::3] == 2).all()


# ---------------------------------------------------------------------------
# greedy rows: the resident kernel's penalised mode (kResGreedyPen)

@pytest.mark.parametrize("pen", [1.3, 0.8, 2.0])
def test_greedy_random_histories(sampler, pen):
    from nimbus_sampler import workloads
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(int(pen * 1000)))
    x = workloads.headline(B)
    gen = [rnd.integers(0, V + 8, size=int(rnd.integers(0, 400))) for _ in range(B)]
    _check(sampler, x, V, _params(temperature=0.0, repetition_penalty=pen), gen,
           f"greedy random pen={pen}")


@pytest.mark.parametrize("pen", [1.0001, 1.3, 0.7])
def test_greedy_histories_on_the_top(sampler, pen):
    # the history holds each row's top tokens: the answer moves to the best
    # unpenalised token or stays on a penalised one, depending on the penalty
    from nimbus_sampler import workloads
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(3 + int(pen * 10)))
    x = workloads.headline(B)
    x[: B // 2] -= 30.0  # rows of negative logits: the penalty multiplies them
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [order[r, : int(rnd.integers(1, 40))] for r in range(B)]
    gpu, _ = _check(sampler, x, V, _params(temperature=0.0, repetition_penalty=pen), gen,
                    f"greedy top pen={pen}")
    on_pen = sum(int(gpu[0][r]) in set(gen[r].tolist()) for r in range(B))
    print(f"[penalty] greedy rows answered by a penalised token: {on_pen}/{B}", flush=True)


def test_greedy_ties_between_penalised_and_plain_values(sampler):
    # logits on a 1/8 lattice, row max m > 0.  Odd rows: six more elements
    # set to 2m and penalised (2m / 2 == m exactly), tying with the plain
    # maxima.  Rows r % 4 == 0: the same six set to m and penalised (m / 2),
    # plus index 0 set to 2m and penalised: a penalised tie at index 0.
    # Other rows: no history.  The lowest index of the f64 maximum must win.
    B, V = 32, 50257
    rnd = np.random.Generator(np.random.PCG64(19))
    x = np.round(rnd.standard_normal((B, V)) * 16.0).astype(np.float32) / np.float32(8.0)
    gen = []
    for r in range(B):
        m = float(x[r].max())
        cand = rnd.choice(np.arange(1, V), size=6, replace=False)
        if r % 2:
            x[r, cand] = np.float32(2.0 * m)
            gen.append(cand)
        elif r % 4 == 0:
            x[r, cand] = np.float32(m)
            x[r, 0] = np.float32(2.0 * m)
            gen.append(np.concatenate([cand, [0]]))
        else:
            gen.append(np.array([], np.int64))
    gpu, _ = _check(sampler, x, V, _params(temperature=0.0, repetition_penalty=2.0), gen,
                    "greedy ties")
    assert all(int(gpu[0][r]) == 0 for r in range(0, B, 4))


def test_greedy_penalised_rows_of_minus_infinity(sampler):
    # Rows of -inf with a history (sampler.rs:172-181): nothing exceeds
    # work[0], so the answer is index 0 whatever the history holds, also
    # when the row is all -inf but one finite element past the history, and
    # when a penalised -inf sits below an unpenalised finite max.
    B, V = 6, 50257
    x = np.full((B, V), -np.inf, np.float32)
    x[2, 9000] = np.float32(-3.0)     # the only finite value, not penalised
    x[3, 5] = np.float32(4.0)         # the only finite value, penalised
    x[4, 40000] = np.float32(1.0)     # finite, and a penalised -inf before it
    gen = [np.array([5]), np.array([5, 17, 50000]), np.array([5]), np.array([5]),
           np.array([3, 7]), np.array([], np.int64)]
    gpu, _ = _check(sampler, x, V, _params(temperature=0.0, repetition_penalty=1.5), gen,
                    "greedy all -inf")
    assert gpu[0].tolist() == [0, 0, 9000, 5, 40000, 0], gpu[0].tolist()


@pytest.mark.parametrize("T,p", [(0.0, 1.0), (0.8, 1.0), (0.8, 0.9), (0.8, 0.97)])
def test_non_finite_and_long_histories_fall_back(sampler, T, p):
    # NaN among the penalised logits, and histories past 4096 ids: declined,
    # recomputed by the general path (kernel == 2), same answers; greedy,
    # top-p off, sparse and dense top-p
    from nimbus_sampler import workloads
    B, V = 4, 50257
    x = workloads.headline(B)
    x[1, 77] = np.float32(np.nan)
    gen = [np.arange(10), np.array([77, 5]), np.arange(5000) % V, np.array([], np.int64)]
    ids, off = _csr(gen)
    params = _params(temperature=T, top_p=p, repetition_penalty=1.5)
    gpu = run_gpu(sampler, x, V, params, list(range(B)), ids, off)
    ref = run_oracle(x, V, params, list(range(B)), ids, off)
    # the NaN row: token and RNG state only, as for every non-finite row (its
    # statistics follow no reference value)
    assert gpu[0][1] == ref[0][1] and np.array_equal(gpu[2][1], ref[2][1])
    keep = [0, 2, 3]
    compare((gpu[0][keep], gpu[1][keep], gpu[2][keep]), (ref[0][keep], ref[1][keep], ref[2][keep]),
            greedy=params.greedy())
    st = gpu[1]
    assert list(st["kernel"]) == [1, 2, 2, 1], st["kernel"]


# ---------------------------------------------------------------------------
# top-p off: the resident kernel's penalised mode (kResAllPen)

@pytest.mark.parametrize("pen,T", [(1.3, 0.8), (0.8, 1.0), (2.0, 0.5), (1.01, 1.3)])
def test_top_p_off_random_histories(sampler, pen, T):
    from nimbus_sampler import workloads
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(int(pen * 100) + int(T * 10)))
    x = workloads.headline(B)
    gen = [rnd.integers(0, V + 8, size=int(rnd.integers(0, 400))) for _ in range(B)]
    _check(sampler, x, V, _params(temperature=T, top_p=1.0, repetition_penalty=pen), gen,
           f"top-p off pen={pen} T={T}")


@pytest.mark.parametrize("pen", [1.0001, 0.5])
def test_top_p_off_histories_on_the_top(sampler, pen):
    # the history holds each row's top tokens: with penalty < 1 their values
    # rise past the row's unpenalised max (the reference moves up with them)
    from nimbus_sampler import workloads
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(23 + int(pen * 10)))
    x = workloads.headline(B)
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [order[r, : int(rnd.integers(1, 60))] for r in range(B)]
    gpu, _ = _check(sampler, x, V, _params(temperature=0.8, top_p=1.0, repetition_penalty=pen),
                    gen, f"top-p off top pen={pen}")
    drew = sum(int(gpu[0][r]) in set(gen[r].tolist()) for r in range(B))
    print(f"[penalty] top-p off rows that drew a penalised token: {drew}/{B}", flush=True)
    assert drew > B // 4


# ---------------------------------------------------------------------------
# 0.95 <= top-p < 1: the dense kernel's penalised form

def _rows(kind, B, V=50257):
    from nimbus_sampler import workloads
    if kind == "normal":
        return workloads.headline(B, V)  # N(0, 3^2)
    if kind == "flat":
        return workloads.c5(B, V)        # U(-0.5, 0.5): nearly every token kept
    return workloads.c2(B, V)            # peaks over N(0, 1): cutoff in the noise


@pytest.mark.parametrize("kind,p,pen,T", [
    ("normal", 0.97, 1.3, 0.8), ("normal", 0.99, 0.8, 0.8), ("normal", 0.95, 2.0, 1.0),
    ("flat", 0.99, 1.3, 1.3), ("flat", 0.99, 0.8, 1.0),
    ("peaks", 0.95, 1.3, 1.0), ("peaks", 0.97, 0.8, 1.0),
])
def test_dense_random_histories(sampler, kind, p, pen, T):
    # histories of 0..400 ids with repeats, some past V; the flat rows list
    # their removed side, the peaks rows (cutoff inside the noise) work in
    # registers without a list
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(int(pen * 100) + int(p * 1000)))
    x = _rows(kind, B)
    gen = []
    for r in range(B):
        n = int(rnd.integers(0, 401))
        g = rnd.integers(0, V + 8, size=n)
        if n > 4:
            g[: n // 4] = g[n // 4: 2 * (n // 4)]  # repeats
        gen.append(g)
    _check(sampler, x, V, _params(temperature=T, top_p=p, repetition_penalty=pen), gen,
           f"dense {kind} pen={pen} p={p}")


@pytest.mark.parametrize("kind,pen,p", [("normal", 1.3, 0.97), ("normal", 0.8, 0.99),
                                        ("peaks", 1.5, 0.95), ("flat", 2.0, 0.99)])
def test_dense_histories_on_the_head(sampler, kind, pen, p):
    # the history holds each row's top tokens (up to 1500 of them), so
    # penalised values are kept, fall into the cutoff's bucket, are ranked
    # and drawn; with penalty < 1 they also set the row max
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(31 + int(pen * 100)))
    x = _rows(kind, B)
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [order[r, : int(rnd.integers(1, 1500))] for r in range(B)]
    gpu, _ = _check(sampler, x, V, _params(temperature=1.0, top_p=p, repetition_penalty=pen), gen,
                    f"dense head {kind} pen={pen} p={p}")
    drew = sum(int(gpu[0][r]) in set(gen[r].tolist()) for r in range(B))
    print(f"[penalty] dense rows that drew a penalised token: {drew}/{B}", flush=True)
    assert drew > 0


def test_dense_ties_between_penalised_and_plain_values(sampler):
    # logits on a 1/1024 lattice (a few elements per value); penalty 2 maps
    # a penalised 2v (or v/2 for v <= 0) to exactly v, so penalised and plain
    # values tie in f64 across the whole row and the stable order (value,
    # then index) decides at the cutoff
    B, V = 48, 50257
    rnd = np.random.Generator(np.random.PCG64(13))
    base = np.round(rnd.standard_normal((B, V)) * 1536.0).astype(np.float32) / np.float32(1024.0)
    gen = []
    for r in range(B):
        idx = rnd.choice(V, size=int(rnd.integers(200, 3000)), replace=False)
        pos = base[r, idx] > 0
        base[r, idx[pos]] *= np.float32(2.0)
        base[r, idx[~pos]] *= np.float32(0.5)
        gen.append(idx)
    for p in (0.95, 0.99):
        _check(sampler, base, V, _params(temperature=0.8, top_p=p, repetition_penalty=2.0),
               gen, f"dense ties p={p}")


def test_dense_padded_rows_and_short_vocabularies(sampler):
    # misaligned rows put penalised ids in the partial head and tail slots
    rnd = np.random.Generator(np.random.PCG64(9))
    for V, ld in ((50257, 50261), (256, 259), (1000, 1000), (53245, 53248)):
        B = 16
        x = _rows("normal", B, V)
        gen = [np.concatenate([[0, 1, 2, V - 1, V - 2, V - 3],
                               rnd.integers(0, V, size=int(rnd.integers(0, 40)))])
               for _ in range(B)]
        ids, off = _csr(gen)
        params = _params(temperature=0.8, top_p=0.97, repetition_penalty=1.4)
        print(f"[penalty] dense padded V={V} ld={ld}", flush=True)
        gpu = run_gpu(sampler, x, V, params, list(range(B)), ids, off, ld=ld)
        ref = run_oracle(x, V, params, list(range(B)), ids, off)
        compare(gpu, ref, greedy=False)
        assert (gpu[1]["kernel"] == 1).all() and (gpu[1]["reject"] == 0).all(), (V, ld)


def test_dense_crowded_lane_falls_back_to_the_general_path(sampler):
    # the dense kernel parks each lane's penalised logits (at most 16 per
    # lane, the lane's slots being 4 (64 k + l) .. + 3 of its wave's range): a
    # history covering every element of one lane's slots declines the row,
    # and the general path recomputes it with the same result
    B, V = 8, 50257
    x = _rows("normal", B)
    crowded = np.array([256 * k + q for k in range(13) for q in range(4)])
    gen = [crowded if r % 2 else np.arange(40000, 40016) for r in range(B)]
    gpu, _ = _check(sampler, x, V, _params(temperature=0.8, top_p=0.97, repetition_penalty=1.3),
                    gen, "dense crowded", on_kernel=False)
    st = gpu[1]
    assert (st["kernel"][0::2] == 1).all() and (st["reject"][0::2] == 0).all()
    assert (st["kernel"][1::2] == 2).all()


@pytest.mark.parametrize("pen,T,p,on", [(0.5, 0.3, 0.99, True), (5.0, 1.7, 0.95, True),
                                        (0.25, 1.0, 0.97, True), (0.8, 0.5, 0.99, True)])
def test_dense_strong_penalties(sampler, pen, T, p, on):
    # penalties far from 1 at low and high temperature: with penalty < 1 the
    # penalised head rises octaves above the unpenalised max (the wave's
    # reference moves past it after the stream), with 5 it sinks into the
    # tail; each row's history mixes its top tokens and random ones.  At
    # penalty 0.5 and T = 0.3 (and in some rows at 0.25 and T = 1) the head
    # rises more than 64 octaves above a wave's first reference (at T = 0.3
    # a logit of 12 is 58 octaves, its penalised value 115): the histogram
    # ring cannot span that, so such a row runs a second time with every
    # first reference raised to 63 octaves below the row max, and stays on
    # the kernel.
    B, V = 64, 50257
    rnd = np.random.Generator(np.random.PCG64(int(pen * 100) + int(T * 10)))
    x = _rows("normal", B)
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [np.concatenate([order[r, : int(rnd.integers(1, 200))], rnd.integers(0, V, size=100)])
           for r in range(B)]
    gpu, _ = _check(sampler, x, V, _params(temperature=T, top_p=p, repetition_penalty=pen), gen,
                    f"dense strong pen={pen} T={T} p={p}", on_kernel=on)
    if not on:
        st = gpu[1]
        assert ((st["kernel"] == 1) | (st["reject"] == 2)).all(), (st["kernel"].tolist(), st["reject"].tolist())
    drew = sum(int(gpu[0][r]) in set(gen[r].tolist()) for r in range(B))
    print(f"[penalty] dense strong pen={pen}: rows that drew a penalised token {drew}/{B}", flush=True)


@pytest.mark.parametrize("V,k,p", [(100000, 0, 0.65), (100000, 0, 1.0), (151936, 0, 0.9),
                                   (50257, 40, 0.9), (100000, 5000, 1.0)])
def test_penalised_masked_rows_on_the_general_path(sampler, V, k, p):
    # penalised rows with -inf entries that the general path answers (long
    # rows with a history, top-k with a history): a -inf element's mass is 0
    # (it was NaN in the f64 correction of the penalised mass, which turned
    # the total into NaN and the row into the bad-total path), and the kept
    # count holds only finite survivors, as the reference's filtered row
    # does (a -inf survivor of top-k or of top-p off is not counted)
    B = 6
    rnd = np.random.Generator(np.random.PCG64(V + k))
    x = (rnd.standard_normal((B, V)) * 0.3).astype(np.float32)
    for r in range(B):
        x[r, rnd.random(V) < rnd.uniform(0.1, 0.9)] = -np.inf
    x[5, :] = -np.inf
    x[5, 123] = 0.5  # one finite element
    gen = [rnd.integers(0, V + 16, size=int(rnd.integers(1, 600))) for _ in range(B)]
    gpu, ref = _check(sampler, x, V, _params(temperature=1.9, top_p=p, top_k=k, repetition_penalty=1.119),
                      gen, f"masked general V={V} k={k} p={p}", on_kernel=False)
    assert (ref[1]["path"] == 4).all()
    assert np.array_equal(gpu[1]["kept"], ref[1]["kept"])
