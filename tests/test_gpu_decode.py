"""GPU parity of nis_decode_step: the batched decode loop of
Engine::generate_ids (engine.rs:279-287) with the model step replaced by
seeded synthetic logits, against the same loop over the CPU oracle's sample().

Each sequence keeps its history on the device (it is also the penalty list,
as `generated` is in the reference), stops on a stop id or on its budget,
and is skipped once done (no token, RNG not advanced).
"""
import numpy as np
import pytest

from parity_util import BOUNDARY

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    import nimbus_sampler as ns
    s = ns.Sampler(0)
    yield s
    s.close()


def _run(sampler, B, V, steps, cap, params_kw, seed, kernels=None, sigma=2.0):
    import torch
    import nimbus_sampler as ns
    from oracle import oracle

    rnd = np.random.Generator(np.random.PCG64(seed))
    seeds = list(range(500, 500 + B))
    max_new = rnd.integers(0, steps + 1, size=B).astype(np.int32)
    max_new[:3] = [0, 1, steps]
    stop = rnd.choice(V, size=3, replace=False).astype(np.uint32)
    logits = (rnd.standard_normal((steps, B, V), dtype=np.float32) * np.float32(sigma))
    # plant a stop id on top of some rows at some steps, so sequences stop early
    for s in range(steps):
        rows = rnd.choice(B, size=B // 6, replace=False)
        logits[s, rows, stop[s % 3]] += np.float32(14.0)

    dev = torch.device("cuda:0")
    params = ns.SamplingParams(**params_kw)
    states = torch.from_numpy(ns.rng_states(seeds).view(np.int64)).to(dev)
    # one sentinel row past the B histories, and every unused slot, must stay untouched
    SENT = 0x7F7F7F7F
    gen_buf = torch.full((B + 1, cap), SENT, dtype=torch.int32, device=dev)
    gen_ids = gen_buf[:B]
    gen_len = torch.zeros(B, dtype=torch.int32, device=dev)
    maxn = torch.from_numpy(max_new).to(dev)
    done = torch.from_numpy((max_new <= 0).astype(np.uint8)).to(dev)
    stop_d = torch.from_numpy(stop.view(np.int32)).to(dev)
    tokens = torch.full((B,), -1, dtype=torch.int32, device=dev)
    gpu_tokens = []
    stats = torch.zeros((B, 64), dtype=torch.uint8, device=dev)
    for s in range(steps):
        tokens.fill_(-1)
        stats.zero_()
        x = torch.from_numpy(np.ascontiguousarray(logits[s])).to(dev)
        sampler.decode_step(x, params, states, gen_ids, gen_len, maxn, done, stop_d, tokens=tokens,
                            stats=stats)
        t = tokens.cpu().numpy().view(np.uint32).copy()
        gpu_tokens.append(t)
        if kernels is not None:  # (kernel, reject) of every row that sampled
            st = ns.stats_view(stats)
            ran = t != 0xFFFFFFFF
            kernels.append((st["kernel"][ran].copy(), st["reject"][ran].copy()))
    torch.cuda.synchronize()
    g_len = gen_len.cpu().numpy()
    g_buf = gen_buf.cpu().numpy()
    g_ids = g_buf[:B].view(np.uint32)
    assert (g_buf[B] == SENT).all(), "history write past the last row"
    for b in range(B):
        assert (g_buf[b, g_len[b]:] == SENT).all(), (b, "history slot past gen_len written")
    assert (g_len <= cap).all(), "history longer than its capacity"
    g_done = done.cpu().numpy()
    g_states = states.cpu().numpy().view(np.uint64)

    p = oracle.make_params(params.temperature, params.top_p, params.top_k,
                           params.repetition_penalty)
    diverged = 0
    for b in range(B):
        rng = oracle.Rng(seeds[b])
        generated = []
        fin = max_new[b] <= 0
        ok = True
        for s in range(steps):
            if fin:
                assert gpu_tokens[s][b] == 0xFFFFFFFF, (b, s, "done row got a token")
                continue
            tok, st = oracle.sample(logits[s, b], p, generated, rng)
            if gpu_tokens[s][b] != tok:
                # allowed only on the oracle's own top-p / CDF boundary; the
                # histories differ from there on, so the row is not compared further
                assert params.temperature > 0.0 and \
                    min(st["topp_margin"], st["cdf_margin"]) <= BOUNDARY, \
                    (b, s, gpu_tokens[s][b], tok)
                ok = False
                diverged += 1
                break
            generated.append(tok)
            fin = tok in set(stop.tolist()) or len(generated) >= max_new[b] or len(generated) >= cap
        if not ok:
            continue
        assert g_len[b] == len(generated), (b, g_len[b], len(generated))
        assert list(g_ids[b, :g_len[b]]) == generated, b
        assert bool(g_done[b]) == fin, (b, g_done[b], fin)
        assert np.array_equal(g_states[b], np.array(rng.words(), dtype=np.uint64)), b
    return diverged, int(g_done.sum()), int((g_len > 0).sum()), int((g_len == cap).sum())


@pytest.mark.parametrize("V,kw,cap", [
    (4096, dict(temperature=0.9, top_p=0.9, repetition_penalty=1.3), 8),
    (4096, dict(temperature=0.7, top_k=40, repetition_penalty=0.8), 8),
    (50257, dict(temperature=0.8, top_p=0.9), 8),
    (50257, dict(temperature=0.0, repetition_penalty=1.2), 8),
    # histories smaller than the steps: a full history ends the sequence
    (4096, dict(temperature=0.9, top_p=0.9, repetition_penalty=1.3), 3),
    (50257, dict(temperature=0.8, top_p=0.9), 3),
    # rows longer than the registers (the long-row kernel, whose penalised
    # rows are finished by the general path through the pending launch)
    (128256, dict(temperature=0.8, top_p=0.9, repetition_penalty=1.3), 8),
    # no penalty: the single-read long kernel (top-p < 0.95)
    (128256, dict(temperature=0.8, top_p=0.9), 5),
    (128256, dict(temperature=0.0, repetition_penalty=1.2), 3),
    (128256, dict(temperature=0.8, top_p=1.0, repetition_penalty=0.8), 8),
])
def test_decode_steps_match_oracle_loop(sampler, V, kw, cap):
    diverged, n_done, n_started, n_full = _run(sampler, B=24, V=V, steps=7, cap=cap,
                                               params_kw=kw, seed=V + int(10 * kw["temperature"]))
    print(f"[decode] V={V} {kw} cap={cap} diverged_at_boundary={diverged} done={n_done} "
          f"started={n_started} full={n_full}", flush=True)
    assert diverged <= 1
    assert n_done > 0 and n_started > 0
    if cap < 7:
        assert n_full > 0, "no history reached its capacity"


@pytest.mark.parametrize("pen,T,p", [(1.3, 0.8, 0.9), (0.8, 0.8, 0.9), (1.2, 0.0, 0.9),
                                     (1.2, 0.8, 1.0), (1.3, 0.8, 0.97)])
def test_penalised_decode_stays_on_the_register_kernels(sampler, pen, T, p):
    # V = 50257, top-p 0.9 / 0.97 (or greedy, or top-p off) with a penalty,
    # logits of the headline's spread (N(0, 3^2)): every step of every
    # sequence runs in the sparse, dense or resident kernel with its history
    # applied in registers
    kernels = []
    kw = dict(temperature=T, top_p=p, repetition_penalty=pen)
    diverged, n_done, n_started, _ = _run(sampler, B=24, V=50257, steps=7, cap=8, params_kw=kw,
                                          seed=77, kernels=kernels, sigma=3.0)
    assert diverged <= 1 and n_started > 0
    k = np.concatenate([a for a, _ in kernels])
    r = np.concatenate([b for _, b in kernels])
    print(f"[decode] penalty {pen} T={T} p={p}: {k.size} row-steps, kernels {np.unique(k).tolist()}, "
          f"rejects {np.unique(r).tolist()}", flush=True)
    assert k.size > 0 and (k == 1).all() and (r == 0).all()


def test_decode_step_rejects_bad_arguments(sampler):
    import ctypes
    import torch
    import nimbus_sampler as ns
    dev = torch.device("cuda:0")
    x = torch.zeros((2, 300), dtype=torch.float32, device=dev)
    st = torch.zeros((2, 4), dtype=torch.int64, device=dev)
    ids = torch.zeros((2, 4), dtype=torch.int32, device=dev)
    n = torch.zeros(2, dtype=torch.int32, device=dev)
    d = torch.zeros(2, dtype=torch.uint8, device=dev)
    p = ns.SamplingParams().to_c()
    L = ns.load_library()
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    base = [sampler._ctx, ptr(x), 300, 2, 300, ctypes.byref(p), ptr(st), ptr(ids)]
    # gen_cap 0, a missing length array, a negative stop count
    assert L.nis_decode_step(*base, 0, ptr(n), ptr(n), None, 0, ptr(d), ptr(n), None) == ns.NIS_EINVAL
    assert L.nis_decode_step(*base, 4, None, ptr(n), None, 0, ptr(d), ptr(n), None) == ns.NIS_EINVAL
    assert L.nis_decode_step(*base, 4, ptr(n), ptr(n), None, -1, ptr(d), ptr(n), None) == ns.NIS_EINVAL
    assert L.nis_decode_step(*base, 4, ptr(n), ptr(n), None, 2, ptr(d), ptr(n), None) == ns.NIS_EINVAL


def test_graph_replays_match_eager_calls(sampler):
    # sample_batch and decode_step captured in a HIP graph: every replay, with
    # eager work and synchronizations between replays, matches the eager call
    # sequence (tokens, RNG states, histories, lengths, flags)
    import torch
    import nimbus_sampler as ns
    from nimbus_sampler import workloads
    dev = torch.device("cuda:0")
    w = workloads.WORKLOADS["headline"]
    B, V, cap = 64, w.V, 8
    x = torch.from_numpy(w.make(w.B)[:B].copy()).to(dev)
    params = ns.SamplingParams(temperature=w.temperature, top_p=w.top_p)
    seeds = list(range(B))

    def fresh():
        return dict(st=torch.from_numpy(ns.rng_states(seeds).view(np.int64)).to(dev),
                    ids=torch.zeros((B, cap), dtype=torch.int32, device=dev),
                    n=torch.zeros(B, dtype=torch.int32, device=dev),
                    mx=torch.full((B,), 5, dtype=torch.int32, device=dev),
                    d=torch.zeros(B, dtype=torch.uint8, device=dev),
                    tok=torch.zeros(B, dtype=torch.int32, device=dev),
                    tok2=torch.zeros(B, dtype=torch.int32, device=dev))

    def step(s):
        sampler.sample_batch(x, params, s["st"], tokens=s["tok"])
        sampler.decode_step(x, params, s["st"], s["ids"], s["n"], s["mx"], s["d"], tokens=s["tok2"])

    def snap(s):
        return [t.clone().cpu() for t in (s["tok"], s["tok2"], s["st"], s["ids"], s["n"], s["d"])]

    eager = fresh()
    ref = []
    for _ in range(3):
        step(eager)
        torch.cuda.synchronize()
        ref.append(snap(eager))
    # each step advances the states, so a replay that re-ran stale work would differ
    assert not torch.equal(ref[0][2], ref[1][2]) and not torch.equal(ref[1][2], ref[2][2])

    g_state = fresh()
    graph = torch.cuda.CUDAGraph()
    cap_stream = torch.cuda.Stream()
    cap_stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap_stream):
        with torch.cuda.graph(graph, stream=cap_stream):
            step(g_state)
    torch.cuda.current_stream().wait_stream(cap_stream)
    torch.cuda.synchronize()
    for k in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = snap(g_state)
        for a, b in zip(got, ref[k]):
            assert torch.equal(a, b), k
        _ = (x * 2.0).sum().item()  # eager work between replays
        torch.cuda.synchronize()
