"""Seeded sweep over the whole parameter space of sample() against the oracle,
and the edge cases its runs found.

The other GPU tests pin each kernel route with hand-picked rows.  This one
draws 48 cases from a fixed seed and crosses what they keep apart: V across
every route (tiny rows, the register kernels up to 53245, the single-read
and long-row kernels up to 262141, the general path beyond), padded and
misaligned row strides, greedy and sampled temperatures, top-k (0, small,
large, V - 1, V), top-p (off, 0, 0.3-0.999), repetition penalties below and
above 1 with histories that hit the row's head, repeat ids and run past V,
and rows that are normal, peaked, flat, on a coarse value lattice (ties) or
partly masked with -inf, some with NaN or +inf.  Every row must match the
oracle's sample() (src/sampler.rs:163-216, apply_repetition_penalty
sampler.rs:83-101) to the bar of parity_util.compare: bit-exact greedy ids
and RNG states, sampled ids equal outside the oracle's 1e-6 boundary rows,
kept counts, and the drawn token's probability and kept mass within 1e-6.
Rows a kernel declines are recomputed by the general path and checked the
same way; the routes each case took are printed.  112 more cases come from
a wider space (_wide_case), and seeded sweeps cover the other entry points:
nis_decode_step loops against the oracle loop, nis_lm_head_logits against
the f32 bound of exact sums, and nis_sample_one / nis_sample_one_noalloc
against the oracle's sample().
"""
import numpy as np
import pytest

from parity_util import compare, run_gpu, run_oracle

pytestmark = pytest.mark.gpu

N_CASES = 48
N_WIDE = 112


@pytest.fixture(scope="module")
def sampler():
    import nimbus_sampler as ns
    s = ns.Sampler(0)
    yield s
    s.close()


def _pick(g, items, weights):
    w = np.asarray(weights, np.float64)
    return items[int(g.choice(len(items), p=w / w.sum()))]


def _case(i):
    """Parameters, rows and histories of sweep case i (deterministic)."""
    g = np.random.Generator(np.random.PCG64(9000 + i))
    route = _pick(g, ["tiny", "register", "long", "beyond"], [2, 10, 4, 1])
    if route == "tiny":
        V = int(g.integers(1, 256))
    elif route == "register":
        V = int(_pick(g, [256, 257, 4099, 50257, 53245, int(g.integers(256, 53246))],
                      [1, 1, 1, 3, 1, 4]))
    elif route == "long":
        V = int(_pick(g, [53246, 128256, 151936, int(g.integers(53246, 262142))], [1, 2, 1, 3]))
    else:
        V = int(g.integers(262142, 300000))
    B = int(_pick(g, [1, 2, 5, 8], [2, 1, 1, 2])) if V > 53245 else int(g.integers(1, 17))
    ld = V + int(_pick(g, [0, 1, 2, 3, 5], [4, 1, 1, 1, 1]))

    kind = _pick(g, ["normal", "peaked", "flat", "lattice", "masked"], [4, 2, 1, 2, 1])
    sigma = float(_pick(g, [0.3, 1.0, 3.0, 8.0], [1, 2, 3, 1]))
    x = (g.standard_normal((B, V)) * sigma).astype(np.float32)
    if kind == "peaked":
        for r in range(B):
            n = int(g.integers(1, 6))
            x[r, g.choice(V, size=min(n, V), replace=False)] += g.uniform(6.0, 15.0, size=min(n, V)).astype(np.float32)
    elif kind == "flat":
        x = g.uniform(-0.5, 0.5, size=(B, V)).astype(np.float32)
    elif kind == "lattice":
        x = (np.round(x * 4.0) / 4.0).astype(np.float32)
    elif kind == "masked":
        for r in range(B):
            m = g.random(V) < g.uniform(0.1, 0.9)
            x[r, m] = -np.inf
    if g.random() < 0.15:  # a non-finite row
        r = int(g.integers(0, B))
        x[r, int(g.integers(0, V))] = np.float32(_pick(g, [np.nan, np.inf, -np.inf], [1, 1, 1]))

    T = 0.0 if g.random() < 0.15 else float(np.exp(g.uniform(np.log(0.1), np.log(2.0))))
    u = g.random()
    top_p = 1.0 if u < 0.25 else (0.0 if u < 0.28 else float(g.uniform(0.3, 0.999)))
    u = g.random()
    if u < 0.55:
        top_k = 0
    elif u < 0.9:
        top_k = int(g.integers(1, max(2, min(V, 2000))))
    else:
        top_k = int(_pick(g, [max(V - 1, 1), V], [1, 1]))
    pen = 1.0 if g.random() < 0.5 else float(g.uniform(0.6, 2.0))

    gen = []
    for r in range(B):
        if pen == 1.0 and g.random() < 0.5:
            gen.append(np.zeros(0, np.int64))
            continue
        n = int(g.integers(0, 600))
        h = g.integers(0, V + 16, size=n)  # ids past V are ignored by the reference
        if n and g.random() < 0.5:  # part of the row's head
            head = np.argsort(-np.nan_to_num(x[r], nan=-np.inf), kind="stable")[: min(V, 64)]
            h[: min(n, len(head))] = head[: min(n, len(head))]
        if n > 8:
            h[: n // 8] = h[n // 8: 2 * (n // 8)]  # repeats
        gen.append(h.astype(np.int64))
    return dict(V=V, B=B, ld=ld, kind=kind, sigma=sigma, T=T, top_p=top_p, top_k=top_k,
                pen=pen, x=x, gen=gen)


def _wide_case(i):
    """A case of the wider space (deterministic): T down to 0.02, sigma up to
    20, rows shifted by +-30 or +-100, constant rows, lone spikes of 40-80,
    -inf runs over up to 99% of a row, histories past the kernels' 4096 ids,
    B up to 64; at most one non-finite value per case, never a NaN beside an
    active top-k (the reference's sort_unstable_by then meets a comparator
    that NaN makes inconsistent: its k-th value is not pinned)."""
    g = np.random.Generator(np.random.PCG64(1300000 + i))
    route = _pick(g, ["tiny", "register", "long", "beyond"], [1, 12, 4, 1])
    if route == "tiny":
        V = int(g.integers(1, 256))
    elif route == "register":
        V = int(_pick(g, [256, 50257, 53245, int(g.integers(256, 53246))], [1, 4, 1, 6]))
    elif route == "long":
        V = int(_pick(g, [53246, 128256, int(g.integers(53246, 262142))], [1, 2, 3]))
    else:
        V = int(g.integers(262142, 330000))
    B = int(g.integers(1, 9)) if V > 53245 else int(_pick(g, [1, 4, 16, 64], [2, 2, 2, 1]))
    ld = V + int(_pick(g, [0, 1, 2, 3, 7], [4, 1, 1, 1, 1]))
    sigma = float(np.exp(g.uniform(np.log(0.2), np.log(20.0))))
    x = (g.standard_normal((B, V)) * sigma).astype(np.float32)
    kinds = []
    if g.random() < 0.3:
        kinds.append("peaks")
        for r in range(B):
            n = min(int(g.integers(1, 20)), V)
            x[r, g.choice(V, size=n, replace=False)] += g.uniform(3.0, 40.0, size=n).astype(np.float32)
    if g.random() < 0.25:
        kinds.append("lattice")
        q = float(_pick(g, [0.0625, 0.25, 1.0], [1, 1, 1]))
        x = (np.round(x / q) * q).astype(np.float32)
    if g.random() < 0.2:
        kinds.append("mask")
        for r in range(B):
            x[r, g.random(V) < g.uniform(0.0, 0.99)] = -np.inf
    if g.random() < 0.1:
        kinds.append("flat")
        x = g.uniform(-0.5, 0.5, size=(B, V)).astype(np.float32)
    if g.random() < 0.12:
        kinds.append("shift")
        x = (x + np.float32(_pick(g, [-100.0, -30.0, 30.0, 100.0], [1, 1, 1, 1]))).astype(np.float32)
    if g.random() < 0.04:
        kinds.append("const")
        x[:] = np.float32(g.uniform(-5, 5))
    if g.random() < 0.08:
        kinds.append("spike")
        for r in range(B):
            x[r, int(g.integers(0, V))] = np.float32(g.uniform(40.0, 80.0))
    if g.random() < 0.08:
        kinds.append("special")
        r = int(g.integers(0, B))
        x[r, int(g.integers(0, V))] = np.float32(_pick(g, [np.nan, np.inf, -np.inf], [1, 1, 1]))
    T = 0.0 if g.random() < 0.12 else float(np.exp(g.uniform(np.log(0.02), np.log(2.5))))
    u = g.random()
    top_p = 1.0 if u < 0.25 else (0.0 if u < 0.29 else (float(g.uniform(0.9, 0.9999)) if u < 0.55
                                                        else float(g.uniform(0.05, 0.9))))
    u = g.random()
    top_k = 0 if u < 0.55 else (int(g.integers(1, max(2, min(V, 3000)))) if u < 0.9
                                else int(_pick(g, [max(V - 1, 1), V, int(g.integers(1, V + 1))], [1, 1, 1])))
    if 0 < top_k < V and np.isnan(x).any():
        x[np.isnan(x)] = np.float32(np.inf)
    pen = 1.0 if g.random() < 0.45 else float(np.exp(g.uniform(np.log(0.5), np.log(2.5))))
    gen = []
    for r in range(B):
        if g.random() < 0.3:
            gen.append(np.zeros(0, np.int64))
            continue
        n = int(_pick(g, [int(g.integers(0, 300)), int(g.integers(300, 6000))], [4, 1]))
        h = g.integers(0, V + 16, size=n)
        if n and g.random() < 0.5:
            head = np.argsort(-np.nan_to_num(x[r], nan=-np.inf), kind="stable")[: min(V, 200)]
            m = min(n, len(head), int(g.integers(1, 201)))
            h[:m] = head[:m]
        gen.append(h.astype(np.int64))
    return dict(V=V, B=B, ld=ld, kind="+".join(kinds) or "normal", sigma=sigma, T=T, top_p=top_p,
                top_k=top_k, pen=pen, x=x, gen=gen)


def _csr(gen):
    off = np.zeros(len(gen) + 1, np.int64)
    off[1:] = np.cumsum([len(h) for h in gen])
    ids = np.concatenate(gen).astype(np.uint32) if off[-1] else np.zeros(0, np.uint32)
    return ids, off


def _check_case(sampler, i, c):
    import nimbus_sampler as ns
    params = ns.SamplingParams(temperature=c["T"], top_p=c["top_p"], top_k=c["top_k"],
                               repetition_penalty=c["pen"])
    ids, off = _csr(c["gen"])
    if ids.size == 0:  # no history at all: neither array is passed (the ABI takes both or none)
        ids = off = None
    print(f"[sweep {i}] B={c['B']} V={c['V']} ld={c['ld']} {c['kind']} sigma={c['sigma']} "
          f"T={c['T']:.4g} top_p={c['top_p']:.4g} top_k={c['top_k']} pen={c['pen']:.4g} "
          f"n_ids={0 if ids is None else len(ids)}", flush=True)
    seeds = [1000 * i + r for r in range(c["B"])]
    gpu = run_gpu(sampler, c["x"], c["V"], params, seeds, ids, off, ld=c["ld"])
    ref = run_oracle(c["x"], c["V"], params, seeds, ids, off)
    rep = compare(gpu, ref, greedy=params.greedy())
    st = gpu[1]
    routes = {f"kernel{k}/reject{r}": int(((st["kernel"] == k) & (st["reject"] == r)).sum())
              for k, r in sorted(set(zip(st["kernel"].tolist(), st["reject"].tolist())))}
    print(f"[sweep {i}] routes {routes} -> {rep}", flush=True)


@pytest.mark.parametrize("i", range(N_CASES))
def test_sweep_case(sampler, i):
    _check_case(sampler, i, _case(i))


@pytest.mark.parametrize("i", range(N_WIDE))
def test_wide_sweep_case(sampler, i):
    _check_case(sampler, i, _wide_case(i))


@pytest.mark.parametrize("i", range(24))
def test_decode_sweep_case(sampler, i):
    # nis_decode_step over 2-8 steps against the oracle loop (histories, stop
    # ids, budgets, RNG states), parameters drawn per case
    import test_gpu_decode as D
    g = np.random.Generator(np.random.PCG64(777000 + i))
    V = int(g.choice([300, 4099, 50257, 53245, 60000, 128256]))
    B = int(g.choice([3, 7, 33])) if V <= 53245 else int(g.choice([3, 5]))
    steps = int(g.integers(2, 9))
    cap = int(g.choice([4, 16, 64]))
    T = 0.0 if g.random() < 0.2 else float(np.exp(g.uniform(np.log(0.1), np.log(2.0))))
    u = g.random()
    top_p = 1.0 if u < 0.3 else (0.0 if u < 0.33 else float(g.uniform(0.3, 0.999)))
    top_k = 0 if g.random() < 0.6 else int(g.integers(1, 2000))
    pen = 1.0 if g.random() < 0.35 else float(np.exp(g.uniform(np.log(0.6), np.log(2.5))))
    sigma = float(g.choice([0.5, 2.0, 5.0]))
    kw = dict(temperature=T, top_p=top_p, top_k=top_k, repetition_penalty=pen)
    print(f"[decode sweep {i}] B={B} V={V} steps={steps} cap={cap} {kw} sigma={sigma}", flush=True)
    D._run(sampler, B, V, steps, cap, kw, 9000 + i, sigma=sigma)


@pytest.mark.parametrize("i", range(32))
def test_lm_head_sweep_case(sampler, i):
    # nis_lm_head_logits on drawn shapes, formats and group sizes, every logit
    # within the f32 bound of its exact sum
    import test_gpu_lm_head as LH
    g = np.random.Generator(np.random.PCG64(31337 + i))
    fmt = int(g.choice([0, 8, 4]))
    H = int(g.choice([64, 96, 128, 200, 256, 384, 512, 768, 1024, 1536, 2048, int(g.integers(2, 1100))]))
    if fmt == 4 and H % 2:
        H += 1
    divs = [d for d in range(1, H + 1) if H % d == 0 and (fmt != 4 or d % 2 == 0)]
    group = None if (fmt == 0 or g.random() < 0.4) else int(g.choice(divs))
    B = int(g.choice([1, 1, 2, 5, 16, 17, 33, 64, 130, 256]))
    V = int(g.choice([1, 7, 100, 1000, 4097, 16384, 50257, int(g.integers(1, 60000))]))
    while B * V * H > 1.5e9:
        V = max(1, V // 2)
    pad_h = int(g.choice([0, 0, 1, 3, 4]))
    pad_v = int(g.choice([0, 0, 1, 5]))
    LH._run(sampler, fmt, B, H, V, group, pad_h, pad_v, seed=i)


@pytest.mark.parametrize("i", range(64))
def test_sample_one_sweep_case(sampler, i):
    # the host drop-in nis_sample_one and its allocation-free twin against
    # the oracle's sample() on one row: same token and advanced state
    import ctypes
    import nimbus_sampler as ns
    from oracle import oracle
    L = ns.load_library()
    g = np.random.Generator(np.random.PCG64(424242 + i))
    V = int(g.choice([1, 2, 9, 255, 256, 4099, 50257, 53245, 60000, 128256, 200003,
                      int(g.integers(1, 262144))]))
    x = (g.standard_normal(V) * float(g.choice([0.5, 2.0, 6.0]))).astype(np.float32)
    if g.random() < 0.2:
        x[g.random(V) < 0.5] = -np.inf
    if g.random() < 0.05:
        x[int(g.integers(0, V))] = np.float32(g.choice([np.inf, -np.inf]))
    T = 0.0 if g.random() < 0.2 else float(np.exp(g.uniform(np.log(0.1), np.log(2.0))))
    u = g.random()
    top_p = 1.0 if u < 0.3 else (0.0 if u < 0.33 else float(g.uniform(0.3, 0.999)))
    top_k = 0 if g.random() < 0.6 else int(g.integers(1, V + 2))
    pen = 1.0 if g.random() < 0.4 else float(np.exp(g.uniform(np.log(0.6), np.log(2.0))))
    gen = g.integers(0, V + 8, size=int(g.integers(0, 300))).astype(np.uint32)
    params = ns.SamplingParams(temperature=T, top_p=top_p, top_k=top_k, repetition_penalty=pen)
    print(f"[one sweep {i}] V={V} T={T:.3g} p={top_p:.4g} k={top_k} pen={pen:.3g} n={gen.size}", flush=True)
    out = []
    for fn in ("nis_sample_one", "nis_sample_one_noalloc"):
        tok = ctypes.c_uint32(0xDEADBEEF)
        st = (ctypes.c_uint64 * 4)(*ns.Rng(99 * i).state())
        p = params.to_c()
        rc = getattr(L, fn)(sampler._ctx, ctypes.c_void_p(x.ctypes.data), V, ctypes.byref(p),
                            ctypes.c_void_p(gen.ctypes.data) if gen.size else None, gen.size, st,
                            ctypes.byref(tok))
        assert rc == ns.NIS_OK, (fn, rc)
        out.append((int(tok.value), [int(v) for v in st]))
    assert out[0] == out[1], out
    rng = oracle.Rng(99 * i)
    ref, ost = oracle.sample(x, oracle.make_params(T, top_p, top_k, pen), gen.tolist(), rng)
    if out[0][0] != ref:  # only on the oracle's own 1e-6 boundary
        assert T > 0 and min(ost["topp_margin"], ost["cdf_margin"]) <= 1e-6, (out[0][0], ref)
    else:
        assert out[0][1] == list(rng.words())


@pytest.mark.parametrize("V", [50257, 128256])
@pytest.mark.parametrize("shift", [-60.0, -200.0])
def test_rows_far_below_zero_with_masked_runs(sampler, V, shift):
    # rows whose values all lie far below 0 (a constant shift leaves the
    # reference's softmax unchanged) with a run of -inf entries: a wave
    # whose first chunk is all -inf used to keep reference 0, so its masses
    # underflowed and its fold floor lay above the searched octaves (the
    # dense and long-row kernels gave wrong kept sets and tokens).  The
    # dense kernel now takes such a wave's first reference from all of its
    # chunks; the long-row kernel declines the row to the general path.
    import nimbus_sampler as ns
    for blk in ((0, 20000), (20000, 40000), (3000, 3600)):
        g = np.random.Generator(np.random.PCG64(int(-shift) + blk[0] + V))
        B = 8
        x = (g.standard_normal((B, V)) + shift).astype(np.float32)
        x[:, blk[0]:blk[1]] = -np.inf
        for T, p, k in ((0.8, 0.9, 0), (0.8, 0.97, 0), (0.8, 1.0, 0), (0.0, 1.0, 0), (0.8, 0.9, 50),
                        (0.3, 0.5, 0)):
            params = ns.SamplingParams(temperature=T, top_p=p, top_k=k)
            print(f"[shifted] V={V} shift={shift} blk={blk} T={T} p={p} k={k}", flush=True)
            gpu = run_gpu(sampler, x, V, params, list(range(B)))
            ref = run_oracle(x, V, params, list(range(B)))
            compare(gpu, ref, greedy=params.greedy())


@pytest.mark.parametrize("pen", [1.0, 0.8, 1.5])
def test_nan_rows_at_top_p_zero(sampler, pen):
    # top-p <= 0 keeps only max_by's entry (sampler.rs:122-134): a NaN hands
    # the running maximum to the entry after it, so the kept entry is the
    # last maximum past the last NaN (or that NaN when it is the last entry),
    # and a finite one is drawn; NaN then survives nothing else
    import nimbus_sampler as ns
    rnd = np.random.Generator(np.random.PCG64(31 + int(pen * 10)))
    for V in (1000, 50257, 100000):
        B = 8
        x = rnd.standard_normal((B, V)).astype(np.float32) * np.float32(2.0)
        x[0, 5] = np.nan                                   # early NaN, the max before it
        x[0, 3] = np.float32(50.0)
        x[1, V - 1] = np.nan                               # NaN last: kept, token 0
        x[2, [10, V // 2]] = np.nan                        # two NaNs
        x[3, 0] = np.nan                                   # NaN at index 0
        x[4, 7] = np.nan
        x[4, V - 3] = np.inf                               # +inf past the NaN
        x[5, V // 3] = np.inf
        x[5, V // 2] = np.nan                              # +inf before the NaN
        x[6, 100] = np.nan
        x[6, 101:] = -np.inf                               # only -inf past the NaN
        x[7, 9] = np.nan
        x[7, [20, 30, 40]] = np.float32(40.0)              # tied maxima past the NaN
        gen = [rnd.integers(0, V, size=50) for _ in range(B)] if pen != 1.0 else None
        ids = off = None
        if gen is not None:
            ids, off = _csr([h.astype(np.int64) for h in gen])
        for T in (0.7, 1.3):
            params = ns.SamplingParams(temperature=T, top_p=0.0, repetition_penalty=pen)
            print(f"[nan p=0] V={V} T={T} pen={pen}", flush=True)
            seeds = list(range(B))
            gpu = run_gpu(sampler, x, V, params, seeds, ids, off)
            ref = run_oracle(x, V, params, seeds, ids, off)
            compare(gpu, ref, greedy=False)


def test_penalised_top_p_off_at_low_temperature(sampler):
    # top-p off with a penalty history at T = 0.06 on a coarse value lattice
    # (sigma 15): a penalised logit's raw value in a wave's first chunk sat
    # ~700 octaves above its penalised value, the wave's reference (which
    # only rises) stayed there and its masses underflowed; such a row is now
    # declined, and the kept mass statistic no longer overflows at large R
    import nimbus_sampler as ns
    rnd = np.random.Generator(np.random.PCG64(74))
    B, V = 16, 50257
    x = (np.round(rnd.standard_normal((B, V)) * 15.0 * 4.0) / 4.0).astype(np.float32)
    order = np.argsort(-x, axis=1, kind="stable")
    gen = [np.concatenate([order[r, : int(rnd.integers(1, 60))], rnd.integers(0, V, size=600)])
           .astype(np.int64) for r in range(B)]
    ids, off = _csr(gen)
    for T, pen in ((0.062, 1.958), (0.1, 1.5), (0.5, 1.3)):
        params = ns.SamplingParams(temperature=T, top_p=1.0, repetition_penalty=pen)
        print(f"[pen low T] T={T} pen={pen}", flush=True)
        gpu = run_gpu(sampler, x, V, params, list(range(B)), ids, off)
        ref = run_oracle(x, V, params, list(range(B)), ids, off)
        compare(gpu, ref, greedy=False)
    # normal rows whose penalised head leads them (sigma 5.4, T 0.126): the
    # wave reference taken from chunk 0's raw logits sat ~55 octaves above the
    # penalised values, and the masses' f32 arguments lost ~1e-6 of precision
    # (the kept mass 2e-6 off); it now starts from the penalised values
    x2 = (rnd.standard_normal((B, V)) * 5.4).astype(np.float32)
    order2 = np.argsort(-x2, axis=1, kind="stable")
    gen2 = [np.concatenate([order2[r, : int(rnd.integers(1, 40))], rnd.integers(0, V, size=400)])
            .astype(np.int64) for r in range(B)]
    ids2, off2 = _csr(gen2)
    for T, pen in ((0.126, 1.3), (0.33, 1.46)):
        params = ns.SamplingParams(temperature=T, top_p=1.0, repetition_penalty=pen)
        print(f"[pen head] T={T} pen={pen}", flush=True)
        gpu = run_gpu(sampler, x2, V, params, list(range(B)), ids2, off2)
        ref = run_oracle(x2, V, params, list(range(B)), ids2, off2)
        rep = compare(gpu, ref, greedy=False)
        assert (gpu[1]["kernel"] == 1).sum() >= B // 2, gpu[1]["kernel"].tolist()  # on the kernel
        print(f"[pen head] -> {rep}", flush=True)
