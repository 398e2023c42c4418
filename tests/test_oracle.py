"""Pins the CPU oracle (oracle/sampler_oracle.c) before anything is compared
against it.

Each check is chosen so that a plausible slip in the restatement (a wrong
constant or shift, `>=` for `>`, inclusive instead of exclusive cumulative
mass, unstable tie order, first instead of last maximum, walking sorted
instead of index order) fails at least one of them:

  - the reference's own unit tests (src/sampler.rs:223-266) as golden vectors;
  - the published SplitMix64(0) stream and an independent Python big-int
    restatement of the RNG (tests/golden/rng_kats.json);
  - GF(2)-linearity of the xoshiro256 state transition;
  - an exact-rational statement of sample() on tiny rows (top-k, top-p,
    penalty, temperature, inverse-CDF walk), compared wherever its decision
    margin exceeds 1e-9 of the mass;
  - the special cases of sample() (non-finite rows, degenerate p, u = 0).
"""
import json
import math
import os
import random
import sys
from fractions import Fraction

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_rng_kats as pyrng  # noqa: E402  independent Python restatement

M64 = (1 << 64) - 1
INF = float("inf")


def f32(v):
    return float(np.float32(v))


# ---------------------------------------------------------------------------
# RNG


def test_rng_seed0_is_splitmix64_outputs_2_to_5(oracle_mod):
    # Published SplitMix64 stream for seed 0 (Steele, Lea & Flood; also the
    # seeding example of the xoshiro authors).
    published = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
                 0xF88BB8A8724C81EC, 0x1B39896A51A8749B]
    assert oracle_mod.Rng(0).words() == published[1:]


def test_rng_matches_python_bigint_kats(oracle_mod):
    doc = json.load(open(os.path.join(HERE, "golden", "rng_kats.json")))
    assert [int(v) for v in doc["splitmix64_seed0_first5"]][0] == 0xE220A8397B1DCDAF
    for k in doc["kats"]:
        r = oracle_mod.Rng(int(k["seed"]))
        assert r.words() == [int(v) for v in k["state"]], k["seed"]
        assert [r.next_u64() for _ in range(8)] == [int(v) for v in k["next_u64"]], k["seed"]
        assert r.words() == [int(v) for v in k["state_after_8"]]
        assert oracle_mod.Rng(int(k["seed"])).next_f64() == float(k["first_f64"])


def test_rng_matches_independent_values(oracle_mod):
    # Values computed independently (a separate big-int restatement of
    # SplitMix64 seeding and xoshiro256++, not this oracle's code).
    table = {
        0: (0x6E789E6AA1B965F4, 0x58F24F57E97E3F07, 0.34744735618868894),
        1: (0xBEEB8DA1658EEC67, 0xFC06D5F275A73FD8, 0.9844793049757329),
        7: (0x044C3CD7F43C661C, 0x237B6A1BEF7875D8, 0.13860190565125818),
        42: (0x28EFE333B266F103, 0xEFDB3ABE2D004720, 0.9369389261528349),
        63: (0x4C7924E17855434F, 0x5DE2DC477B1D3CF3, 0.36674286599292294),
        1000: (0xD07A9D82D4F4BBAF, 0x0BAC1032FC33F4A3, 0.04559422726397577),
        0x5DEECE66D: (0x506E90F594419A89, 0xBBC2027C2A86762D, 0.7334291031970908),
    }
    for seed, (s0, first, f) in table.items():
        r = oracle_mod.Rng(seed)
        assert r.words()[0] == s0
        assert r.next_u64() == first
        assert oracle_mod.Rng(seed).next_f64() == f


def test_rng_is_deterministic_and_seeded(oracle_mod):
    # sampler.rs:230-239
    a, b = oracle_mod.Rng(42), oracle_mod.Rng(42)
    for _ in range(100):
        assert a.next_u64() == b.next_u64()
    c = oracle_mod.Rng(43)
    assert a.next_u64() != c.next_u64()


def test_xoshiro_transition_is_gf2_linear(oracle_mod):
    rnd = random.Random(5)

    def step(words):
        r = oracle_mod.Rng(state=words)
        r.next_u64()
        return r.words()

    for _ in range(50):
        a = [rnd.getrandbits(64) for _ in range(4)]
        b = [rnd.getrandbits(64) for _ in range(4)]
        ab = [x ^ y for x, y in zip(a, b)]
        assert step(ab) == [x ^ y for x, y in zip(step(a), step(b))]


def test_next_f64_is_top_53_bits(oracle_mod):
    for seed in range(20):
        x = oracle_mod.Rng(seed).next_u64()
        u = oracle_mod.Rng(seed).next_f64()
        assert 0.0 <= u < 1.0
        assert u * 2.0**53 == float(x >> 11)


# ---------------------------------------------------------------------------
# Reference unit tests (src/sampler.rs:223-266) as golden vectors


def test_greedy_takes_first_max(oracle_mod):
    p = oracle_mod.make_params(temperature=0.0)
    tok, st = oracle_mod.sample(np.array([0.1, 5.0, 5.0, -1.0], np.float32), p, (),
                                oracle_mod.Rng(0))
    assert tok == 1 and st["path"] == oracle_mod.PATH_GREEDY


def test_top_k_keeps_only_best_k(oracle_mod):
    out = oracle_mod.top_k_filter([1.0, 5.0, 3.0, 4.0], 2)
    assert out.tolist() == [-INF, 5.0, -INF, 4.0]


def test_repetition_penalty_divides_positive_multiplies_negative(oracle_mod):
    out = oracle_mod.apply_repetition_penalty([2.0, -2.0], [0, 1], 2.0)
    assert out.tolist() == [1.0, -4.0]


def test_top_p_zero_keeps_argmax_only(oracle_mod):
    out, _, _ = oracle_mod.top_p_filter([1.0, 5.0, 3.0], 0.0)
    assert out.tolist() == [-INF, 5.0, -INF]


# ---------------------------------------------------------------------------
# Exact-rational statement of sample() for tiny rows.


def exact_sample(x, T, top_k, top_p, penalty, generated, u):
    """Returns (token, kept_indices, min_margin) with exact mass arithmetic.

    Probabilities are glibc exp values (math.exp), then every sum, the top-p
    rule and the walk are evaluated exactly on those rationals."""
    n = len(x)
    work = [float(np.float32(v)) for v in x]
    pen = f32(penalty)
    if pen != 1.0 and generated:
        for i in set(generated):
            if i < n:
                work[i] = work[i] / pen if work[i] > 0 else work[i] * pen
    if f32(T) <= 0.0:
        best = 0
        for i, v in enumerate(work):
            if v > work[best]:
                best = i
        return best, None, INF
    temp = max(f32(T), 1e-6)
    w = [v / temp for v in work]
    margin = INF
    if 0 < top_k < n:
        kth = sorted(w, reverse=True)[top_k - 1]
        w = [v if v >= kth else -INF for v in w]
    p = f32(top_p)
    if p <= 0.0:
        best = max(range(n), key=lambda i: (w[i], i))  # last of the maxima
        w = [w[i] if i == best else -INF for i in range(n)]
    elif p < 1.0:
        order = sorted(range(n), key=lambda i: -w[i])  # Python's sort is stable
        m = w[order[0]]
        E = [Fraction(math.exp(w[i] - m)) for i in order]
        Z = sum(E)
        pz = Fraction(p) * Z
        cum = Fraction(0)
        removed = set()
        for pos, i in enumerate(order):
            D = cum - E[pos]
            if w[i] != -INF:
                margin = min(margin, abs(float((D - pz) / Z)))
            if D > pz:
                removed.add(i)
            cum += E[pos]
        w = [-INF if i in removed else w[i] for i in range(n)]
    m = max(w)
    kept = [i for i in range(n) if w[i] != -INF]
    e = [Fraction(math.exp(v - m)) if v != -INF else Fraction(0) for v in w]
    total = sum(e)
    r = Fraction(u) * total
    acc = Fraction(0)
    tok = n - 1
    for i in range(n):
        before = acc
        acc += e[i]
        if acc >= r:
            tok = i
            margin = min(margin, float((r - before) / total), float((acc - r) / total))
            break
    return tok, kept, margin


def _random_row(rnd, n):
    kind = rnd.random()
    if kind < 0.4:  # coarse lattice: many exact ties
        return [rnd.randint(-8, 8) / 4.0 for _ in range(n)]
    if kind < 0.8:
        return [rnd.gauss(0.0, 2.0) for _ in range(n)]
    return [rnd.uniform(-0.5, 0.5) for _ in range(n)]


def test_sample_matches_exact_statement_on_tiny_rows(oracle_mod):
    rnd = random.Random(1234)
    checked = 0
    for case in range(4000):
        n = rnd.randint(1, 9)
        x = np.array(_random_row(rnd, n), np.float32)
        T = rnd.choice([0.0, 0.25, 0.7, 1.0, 1.6])
        top_k = rnd.choice([0, 0, 1, 2, 3, n])
        top_p = rnd.choice([1.0, 1.0, 0.0, 0.3, 0.5, 0.9, 0.99])
        penalty = rnd.choice([1.0, 1.0, 1.3, 0.7])
        generated = [rnd.randrange(n + 2) for _ in range(rnd.randint(0, 4))]
        seed = rnd.getrandbits(64)
        params = oracle_mod.make_params(T, top_p, top_k, penalty)
        rng = oracle_mod.Rng(seed)
        tok, st = oracle_mod.sample(x, params, generated, rng)
        s = pyrng.rng_new(seed)
        u = (pyrng.next_u64(s) >> 11) / float(1 << 53)
        etok, kept, margin = exact_sample(x, T, top_k, top_p, penalty, generated, u)
        if f32(T) <= 0.0:
            assert tok == etok, (case, x, T)
            assert rng.words() == pyrng.rng_new(seed)  # greedy leaves the RNG alone
            continue
        assert st["u"] == u
        assert rng.words() == s  # exactly one next_u64
        if margin > 1e-9:
            assert tok == etok, (case, x.tolist(), T, top_k, top_p, penalty, generated, u)
            assert st["kept"] == len(kept)
            checked += 1
    assert checked > 2500


def test_top_p_general_rule_examples(oracle_mod):
    # probs ~ [0.6652, 0.2447, 0.0900]: with p=0.5 the second token has
    # cum_excl - q = 0.6652 - 0.2447 = 0.42 <= 0.5 -> kept; the third has
    # 0.9100 - 0.0900 = 0.82 > 0.5 -> removed.  A textbook `cum_excl > p`
    # rule would also remove the second token.
    out, margin, _ = oracle_mod.top_p_filter([2.0, 1.0, 0.0], 0.5)
    assert out.tolist() == [2.0, 1.0, -INF]
    # stable order: equal values keep index order, so of three tied tokens
    # the highest index is removed first
    out, _, _ = oracle_mod.top_p_filter([0.0, 0.0, 0.0], 0.2)
    # probs 1/3 each: pos0 D=-1/3 keep, pos1 D=0 keep, pos2 D=1/3 > 0.2 remove
    assert out.tolist() == [0.0, 0.0, -INF]


def test_walk_is_in_index_order(oracle_mod):
    # token 2 holds most mass but index order puts token 0's mass first
    x = np.array([0.0, -50.0, 3.0], np.float32)
    params = oracle_mod.make_params(1.0, 1.0)
    for seed in range(64):
        rng = oracle_mod.Rng(seed)
        tok, st = oracle_mod.sample(x, params, (), rng)
        e0 = math.exp(0.0 - 3.0)
        expect = 0 if st["u"] * st["z_kept"] <= e0 else 2
        assert tok == expect


# ---------------------------------------------------------------------------
# Special cases of sample()


@pytest.mark.parametrize("row,params,expect_tok,expect_path", [
    ([-INF, -INF, -INF], dict(temperature=1.0, top_p=0.9), 0, 2),
    ([1.0, INF, 2.0, INF], dict(temperature=1.0, top_p=1.0), 1, 2),
    ([1.0, INF, 2.0, INF], dict(temperature=1.0, top_p=0.0), 3, 2),
    ([1.0, INF, 2.0, INF], dict(temperature=1.0, top_p=0.5), 1, 2),
    ([float("nan"), 3.0, 1.0], dict(temperature=0.0), 0, 1),
    ([0.5, float("nan"), 3.0], dict(temperature=0.0), 2, 1),
    ([0.5, float("nan"), 3.0], dict(temperature=1.0, top_p=1.0), 0, 3),
    ([-INF, 2.0, -INF], dict(temperature=1.0, top_p=1.0), 1, 4),
])
def test_special_rows(oracle_mod, row, params, expect_tok, expect_path):
    rng = oracle_mod.Rng(9)
    before = rng.words()
    tok, st = oracle_mod.sample(np.array(row, np.float32), oracle_mod.make_params(**params), (), rng)
    assert tok == expect_tok
    assert st["path"] == expect_path
    assert (rng.words() != before) == (expect_path == oracle_mod.PATH_DRAW)


def test_temperature_clamp_and_nan(oracle_mod):
    x = np.array([0.0, 1e-6, 3e-6], np.float32)
    # T = 1e-9 behaves exactly like T = 1e-6 (sampler.rs:183)
    for T in (1e-9, float("nan")):
        a = oracle_mod.sample(x, oracle_mod.make_params(T, 1.0), (), oracle_mod.Rng(3))
        b = oracle_mod.sample(x, oracle_mod.make_params(1e-6, 1.0), (), oracle_mod.Rng(3))
        assert a[0] == b[0] and a[1]["z_kept"] == b[1]["z_kept"]


def test_zero_draw_returns_index_zero_even_if_filtered():
    # u == 0 makes r == 0, so the walk stops at index 0 (sampler.rs:210-213)
    tok, kept, _ = exact_sample([0.0, 5.0], 1.0, 1, 1.0, 1.0, [], 0.0)
    assert tok == 0 and kept == [1]


# ---------------------------------------------------------------------------
# Batched driver (threads.rs fork-join) == sequential calls


def test_batch_driver_equals_sequential(oracle_mod):
    rnd = np.random.Generator(np.random.PCG64(11))
    B, V = 37, 300
    x = rnd.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    params = oracle_mod.make_params(0.9, 0.8, 0, 1.2)
    gen = [rnd.integers(0, V, size=rnd.integers(0, 6)).astype(np.uint32) for _ in range(B)]
    off = np.zeros(B + 1, np.int64)
    off[1:] = np.cumsum([len(g) for g in gen])
    ids = np.concatenate(gen) if off[-1] else np.zeros(0, np.uint32)
    for threads in (1, 3, 8):
        states = oracle_mod.rng_states(range(B))
        toks, stats, workers = oracle_mod.sample_batch(x, V, params, states, ids, off, threads)
        assert workers == threads
        for b in range(B):
            rng = oracle_mod.Rng(b)
            t, _ = oracle_mod.sample(x[b], params, gen[b], rng)
            assert t == toks[b]
            assert rng.words() == states[b].tolist()


def test_fork_join_covers_every_row_once(oracle_mod):
    # threads.rs:113-135 analogue: every row written exactly once
    B, V = 10003, 2
    x = np.zeros((B, V), np.float32)
    x[np.arange(B), np.arange(B) % 2] = 1.0
    states = oracle_mod.rng_states([0] * B)
    toks, _, _ = oracle_mod.sample_batch(x, V, oracle_mod.make_params(0.0), states, n_threads=7)
    assert np.array_equal(toks, (np.arange(B) % 2).astype(np.uint32))
