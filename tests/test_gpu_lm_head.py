"""GPU parity of nis_lm_head_logits, the logits producer of Model::logits_last
(model.rs:317-325 -> gemv_into, model.rs:65-86; quant.rs:121-161), against
the oracle's exact f64 sums.

Bar: every logit within the f32 error bound of a length-H sum of its exact
value (gamma_{H+2+groups} * sum |x_h w_h|, oracle.lm_head_oracle.f32_bound):
the reference's own f32 SIMD order meets the same bound, and neither order is
the other's.  The padding of a strided output row stays untouched.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    import nimbus_sampler as ns
    s = ns.Sampler(0)
    yield s
    s.close()


def _weights(fmt, V, H, group, rnd):
    from oracle import lm_head_oracle as lh
    w = (rnd.standard_normal((V, H)) * 0.05).astype(np.float32)
    if fmt == lh.FMT_F32:
        return w.reshape(-1), None
    bits = 8 if fmt == lh.FMT_INT8 else 4
    return lh.quantize(w, V, H, bits, group)


def _run(sampler, fmt, B, H, V, group=None, pad_h=0, pad_v=0, seed=0):
    import torch
    from oracle import lm_head_oracle as lh
    rnd = np.random.default_rng(seed)
    x = rnd.standard_normal((B, H)).astype(np.float32)
    data, scales = _weights(fmt, V, H, group, rnd)
    dev = torch.device("cuda:0")
    xb = torch.full((B, H + pad_h), float("nan"), dtype=torch.float32, device=dev)
    xb[:, :H] = torch.from_numpy(x).to(dev)
    out = torch.full((B, V + pad_v), float("nan"), dtype=torch.float32, device=dev)
    d = torch.from_numpy(np.ascontiguousarray(data)).to(dev)
    s = torch.from_numpy(scales).to(dev) if scales is not None else None
    print(f"[lm_head] fmt={fmt} B={B} H={H} V={V} group={group} pad=({pad_h},{pad_v})", flush=True)
    sampler.lm_head_logits(xb[:, :H], fmt, d, V, scales=s, group_size=group or 0, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exact, absd = lh.lm_head_logits(x, fmt, data, scales, V, H, group)
    groups = H // (group or H)
    err = np.abs(got[:, :V].astype(np.float64) - exact)
    bound = lh.f32_bound(absd, H, groups)
    worst = float((err / bound).max())
    assert np.all(err <= bound), f"max err/bound {worst}"
    if pad_v:
        assert np.isnan(got[:, V:]).all(), "padding written"
    return worst


@pytest.mark.parametrize("fmt,B,H,V,group,pad_h,pad_v", [
    (0, 1, 128, 448, None, 0, 0),        # tiny-gpt2 tied head, one decode row
    (0, 3, 96, 12, None, 0, 3),          # the reference's dot_row test shape
    (0, 256, 768, 50257, None, 0, 0),    # GPT-2 head at the headline batch
    (0, 130, 100, 999, None, 3, 5),      # H % 4 != 0 and strided rows: element loads
    (0, 17, 768, 4097, None, 4, 0),      # just past one 16-row tile, ldh % 4 == 0
    (8, 37, 768, 5000, None, 0, 0),      # int8 per row
    (8, 70, 768, 3001, 48, 0, 7),        # int8, groups of 48 (reference test group)
    (8, 9, 96, 130, 6, 0, 0),            # int8, group % 4 != 0: element path
    (4, 5, 128, 1000, 32, 0, 0),         # int4, groups of 32
    (4, 64, 768, 2048, None, 0, 0),      # int4 per row
    (4, 2, 98, 77, 14, 0, 0),            # int4, H % 4 != 0: element path
    (4, 300, 256, 1500, 64, 0, 0),       # int4 grouped, more than one b tile along y
    # one hidden row: the VALU GEMV (16 or 64 lanes per weight row) or, where
    # its shape does not hold, the matrix-core kernel
    (0, 1, 768, 50257, None, 0, 0),      # 64 lanes per row, 3 runs per lane
    (8, 1, 768, 50257, None, 0, 0),      # 16 lanes per row
    (8, 1, 768, 3001, 48, 0, 0),         # groups of 48 = 3 runs of 16
    (4, 1, 768, 50257, 64, 0, 0),        # int4 groups of 64, 48 runs of 16 codes per row
    (4, 1, 4096, 999, None, 0, 0),       # 64 lanes, 4 runs per lane
    (4, 1, 784, 1000, None, 0, 0),       # int4, 49 runs: 16 lanes, 4 runs per lane, some idle
    (8, 1, 1024, 999, None, 0, 0),       # int8, 64 runs: 16 lanes, 4 runs per lane
    (8, 1, 768, 500, 16, 0, 0),          # int8, groups of one run
    (0, 1, 1024, 777, None, 0, 0),       # 64 lanes, 4 runs per lane (the cap)
    (0, 1, 4096, 300, None, 0, 0),       # over the cap: matrix-core kernel
    (8, 1, 96, 130, 8, 0, 0),            # group 8 < run of 16: matrix-core kernel
    (8, 3, 40, 77, 1, 0, 0),             # int8, one scale per weight (group 1)
    (8, 1, 40, 77, 1, 0, 0),             # the same through the one-row dispatch
    (4, 1, 40, 65, None, 0, 0),          # int4 H % 16 != 0: matrix-core kernel
])
def test_lm_head_matches_exact_sum_within_f32_bound(sampler, fmt, B, H, V, group, pad_h, pad_v):
    worst = _run(sampler, fmt, B, H, V, group, pad_h, pad_v, seed=B + H + V)
    print(f"[lm_head] worst err/bound {worst:.3g}", flush=True)


def test_lm_head_rejects_bad_arguments(sampler):
    import torch
    import nimbus_sampler as ns
    dev = torch.device("cuda:0")
    L = ns.load_library()
    x = torch.zeros((2, 6), dtype=torch.float32, device=dev)
    out = torch.zeros((2, 8), dtype=torch.float32, device=dev)
    q = torch.zeros(64, dtype=torch.uint8, device=dev)
    sc = torch.ones(32, dtype=torch.float32, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def call(fmt, group, H=6, V=8, ld=8, scales=sc, ldh=6):
        w = ns.NisWeights(fmt, group, q.data_ptr(), scales.data_ptr() if scales is not None else None)
        return L.nis_lm_head_logits(sampler._ctx, p(x), ldh, 2, H, ctypes.byref(w), V, p(out), ld)

    assert call(ns.W_F32, 2) == ns.NIS_EINVAL          # f32 takes no group
    assert call(ns.W_INT8, 0, scales=None) == ns.NIS_EINVAL
    assert call(ns.W_INT8, 4) == ns.NIS_EINVAL         # 4 does not divide H = 6
    assert call(ns.W_INT4, 0, H=5, ldh=6) == ns.NIS_EINVAL  # odd H for int4
    assert call(ns.W_INT4, 3) == ns.NIS_EINVAL         # odd group for int4
    assert call(ns.W_INT8, 0, ld=7) == ns.NIS_EINVAL   # ld < V
    assert call(ns.W_INT8, 0, ldh=5) == ns.NIS_EINVAL  # ldh < H
    assert call(7, 0) == ns.NIS_EINVAL                 # unknown format


def test_lm_head_feeds_sampler(sampler):
    # hidden -> logits -> token on one stream: the tokens equal the oracle's
    # sample() on the same device logits (boundary rows counted, not failed)
    import torch
    import nimbus_sampler as ns
    from oracle import lm_head_oracle as lh
    from parity_util import compare, run_oracle
    rnd = np.random.default_rng(3)
    B, H, V = 64, 768, 50257
    x = torch.from_numpy(rnd.standard_normal((B, H)).astype(np.float32)).cuda()
    data, scales = _weights(lh.FMT_INT8, V, H, 64, rnd)
    # scale the head so logits span a realistic range (std ~ 3)
    d = torch.from_numpy(data).cuda()
    s = torch.from_numpy(scales * np.float32(2.0)).cuda()
    logits = sampler.lm_head_logits(x, ns.W_INT8, d, V, scales=s, group_size=64)
    params = ns.SamplingParams(temperature=0.8, top_p=0.9)
    seeds = list(range(7, 7 + B))
    st = torch.from_numpy(ns.rng_states(seeds).view(np.int64)).cuda()
    stats = torch.zeros((B, 64), dtype=torch.uint8, device="cuda")
    toks = sampler.sample_batch(logits, params, st, stats=stats)
    torch.cuda.synchronize()
    host = logits.cpu().numpy()
    gpu = (toks.cpu().numpy().astype(np.uint32), ns.stats_view(stats),
           st.cpu().numpy().view(np.uint64))
    rep = compare(gpu, run_oracle(host, V, params, seeds), greedy=False)
    print(f"[lm_head->sample] {rep}", flush=True)


def test_bench_kernel_cli_checks_match_oracle():
    # the reference's bench-kernel workload through the CLI: each y[0] check
    # equals the exact dot of its format within the f32 bound (+ the JSON's
    # 4-decimal rounding)
    from nimbus_sampler import cli
    from oracle import lm_head_oracle as lh
    res = cli.bench_kernel(steps=2, warmup=1)
    print(f"[bench-kernel] {res}", flush=True)
    x, w_f32, w_i8, w_i4 = cli.reference_kernel_inputs()
    ones = np.ones(1, np.float32)
    for fmt, data, check in ((lh.FMT_F32, w_f32[:768], res["checks"][0]),
                             (lh.FMT_INT8, w_i8[:768], res["checks"][1]),
                             (lh.FMT_INT4, w_i4[:384], res["checks"][2])):
        exact, absd = lh.lm_head_logits(x[None, :], fmt, data, ones, 1, 768)
        assert abs(check - exact[0, 0]) <= lh.f32_bound(absd[0, 0], 768) + 5e-5, (fmt, check, exact)
    assert all(res[f"{k}_gflops"] > 0 for k in ("f32", "int8", "int4"))


# ---------------------------------------------------------------------------
# nis_lm_head_greedy: the one-row GEMV with the greedy token fused into its
# epilogue.  The token must be the reference's greedy answer (sampler.rs:172-
# 181: first index of the maximum, a NaN at index 0 gives 0) on the logits
# the same call writes, and equal nis_argmax_batch on them.

def _greedy_ref(v):
    best = 0
    for i in range(1, len(v)):
        if v[i] > v[best]:
            best = i
    return best


def _greedy_case(sampler, fmt, H, V, group=None, seed=0, tweak=None, with_logits=True):
    import torch
    rnd = np.random.default_rng(seed)
    x = rnd.standard_normal(H).astype(np.float32)
    data, scales = _weights(fmt, V, H, group, rnd)
    if tweak is not None:
        data, scales, x = tweak(data, scales, x)
    dev = torch.device("cuda:0")
    d = torch.from_numpy(np.ascontiguousarray(data)).to(dev)
    s = torch.from_numpy(scales).to(dev) if scales is not None else None
    xt = torch.from_numpy(x).to(dev)
    print(f"[lm_head greedy] fmt={fmt} H={H} V={V} group={group} seed={seed}", flush=True)
    logits = torch.full((V,), float("nan"), dtype=torch.float32, device=dev) if with_logits else None
    tok = sampler.lm_head_greedy(xt, fmt, d, V, scales=s, group_size=group or 0, logits=logits)
    # the same head through the two-call path, for the logits and argmax_batch
    out = sampler.lm_head_logits(xt.reshape(1, -1), fmt, d, V, scales=s, group_size=group or 0)
    am = sampler.argmax_batch(out)
    torch.cuda.synchronize()
    lg = out.cpu().numpy()[0]
    if with_logits:
        assert np.array_equal(logits.cpu().numpy(), lg, equal_nan=True), "fused logits differ"
    t = int(tok.cpu().numpy()[0])
    assert t == _greedy_ref(lg) == int(am.cpu().numpy()[0]), (t, _greedy_ref(lg))
    return t


@pytest.mark.parametrize("fmt,H,V,group", [
    (0, 768, 50257, None),    # GPT-2 head, 64 lanes per row
    (8, 768, 50257, None),    # int8, 16 lanes per row
    (8, 768, 50257, 64),      # int8 grouped
    (4, 768, 50257, 64),      # int4 grouped
    (4, 4096, 999, None),     # 64 lanes, 4 runs per lane
    (0, 1024, 777, None),     # a grid of few workgroups, the last one partly past V
    (0, 4096, 300, None),     # over the one-row kernel's cap: the two-launch form
    (4, 40, 65, None),        # int4 H % 16 != 0: the two-launch form
])
def test_greedy_matches_argmax_of_the_logits(sampler, fmt, H, V, group):
    for seed in range(3):
        _greedy_case(sampler, fmt, H, V, group, seed=seed, with_logits=seed != 1)


def test_greedy_ties_take_the_first_index(sampler):
    # duplicated weight rows give bit-identical logits: the lowest index of
    # the maximum must win, across waves and workgroups
    H, V = 768, 50257

    def tweak(data, scales, x):
        w = data.reshape(V, H).copy()
        top = int(np.argmax(w @ x))
        for j in (7, 5000, top + 1 if top + 1 < V else 3, 49999):
            w[j] = w[top]
        w[2] = w[top]  # the lowest copy
        return w.reshape(-1), scales, x
    assert _greedy_case(sampler, 0, H, V, tweak=tweak) == 2


def test_greedy_nan_rules(sampler):
    # a NaN logit at index 0 gives 0 (every comparison fails); a NaN elsewhere
    # never wins
    H, V = 768, 20000

    def nan_at(j):
        def tweak(data, scales, x):
            w = data.reshape(V, H).copy()
            w[j, 5] = np.float32(np.nan)
            return w.reshape(-1), scales, x
        return tweak
    assert _greedy_case(sampler, 0, H, V, tweak=nan_at(0)) == 0
    t = _greedy_case(sampler, 0, H, V, tweak=nan_at(123))
    assert t != 123
