"""GPU-vs-oracle comparison used by the GPU tests (and bench.py's report).

Bar (per row, from the oracle's own margins):
  - greedy / argmax ids: bit-exact;
  - RNG state after the call: bit-exact (advanced once iff a draw happened);
  - sampled ids: equal unless the row is a boundary row, i.e. the oracle's
    top-p decision margin |cum_excl - q - p| or its CDF margin
    |r - prefix| / total is <= 1e-6 (such rows are counted, not failed);
  - kept-set size: equal unless the top-p margin is <= 1e-6;
  - probability of the drawn token and the kept mass: within 1e-6 relative;
  - a sampled-id mismatch is allowed only where the oracle's margin is at
    most 3e-7 (STRICT_BOUNDARY), three times the GPU's measured mass error
    (~1e-7), although any row within 1e-6 is counted as a boundary row.
"""
import numpy as np

BOUNDARY = 1e-6
STRICT_BOUNDARY = 3e-7
PROB_RTOL = 1e-6


def run_gpu(sampler, x, V, params, seeds, gen_ids=None, gen_offsets=None, ld=None):
    """Run nis_sample_batch on a host array; returns (tokens, stats, states)."""
    import torch
    import nimbus_sampler as ns
    B = x.shape[0]
    dev = torch.device("cuda:0")
    if ld is None or ld == x.shape[1]:
        xd = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    else:
        buf = torch.full((B, ld), float("nan"), dtype=torch.float32, device=dev)
        buf[:, :V] = torch.from_numpy(np.ascontiguousarray(x[:, :V])).to(dev)
        xd = buf
    st = torch.from_numpy(ns.rng_states(seeds).view(np.int64)).to(dev)
    stats = torch.zeros((B, 64), dtype=torch.uint8, device=dev)
    gi = go = None
    if gen_ids is not None:
        gi = torch.from_numpy(np.ascontiguousarray(gen_ids, np.uint32).view(np.int32)).to(dev)
        go = torch.from_numpy(np.ascontiguousarray(gen_offsets, np.int64)).to(dev)
    toks = sampler.sample_batch(xd, params, st, V=V, gen_ids=gi, gen_offsets=go, stats=stats)
    torch.cuda.synchronize()
    return (toks.cpu().numpy().astype(np.uint32), ns.stats_view(stats),
            st.cpu().numpy().view(np.uint64))


def run_oracle(x, V, params, seeds, gen_ids=None, gen_offsets=None):
    from oracle import oracle
    p = oracle.make_params(params.temperature, params.top_p, params.top_k,
                           params.repetition_penalty)
    states = oracle.rng_states(seeds)
    toks, stats, _ = oracle.sample_batch(np.ascontiguousarray(x[:, :V]), V, p, states, gen_ids,
                                         gen_offsets)
    return toks, stats, states


def compare(gpu, ref, greedy):
    """Returns a report dict; raises AssertionError on a parity failure."""
    g_tok, g_st, g_states = gpu
    r_tok, r_st, r_states = ref
    B = len(r_tok)
    rej = g_st["reject"][g_st["kernel"] == 2]
    rep = {"rows": B, "fast_rows": int((g_st["kernel"] == 1).sum()),
           "sparse_rows": int(((g_st["kernel"] == 1) & (g_st["reject"] == 0)).sum()),
           "rejects": {int(k): int(n) for k, n in zip(*np.unique(rej, return_counts=True))}}
    assert np.array_equal(g_states, r_states), \
        f"rng state mismatch on rows {np.nonzero((g_states != r_states).any(1))[0][:10].tolist()}"
    if greedy:
        bad = np.nonzero(g_tok != r_tok)[0]
        assert bad.size == 0, f"greedy mismatch rows {bad[:10].tolist()}: gpu {g_tok[bad[:10]]} " \
                              f"ref {r_tok[bad[:10]]}"
        rep["greedy_mismatch"] = 0
        return rep
    topp_b = r_st["topp_margin"] <= BOUNDARY
    cdf_b = r_st["cdf_margin"] <= BOUNDARY
    boundary = topp_b | cdf_b
    mism = g_tok != r_tok
    bad = np.nonzero(mism & ~boundary)[0]
    assert bad.size == 0, (
        f"sampled id mismatch outside boundary rows {bad[:10].tolist()}: gpu {g_tok[bad[:10]]} "
        f"ref {r_tok[bad[:10]]} paths gpu {g_st['path'][bad[:10]]} ref {r_st['path'][bad[:10]]} "
        f"kept gpu {g_st['kept'][bad[:10]]} ref {r_st['kept'][bad[:10]]} "
        f"u gpu {g_st['u'][bad[:10]]} ref {r_st['u'][bad[:10]]}")
    path_bad = np.nonzero((g_st["path"] != r_st["path"]) & ~boundary)[0]
    assert path_bad.size == 0, f"path mismatch rows {path_bad[:10].tolist()}"
    kept_bad = np.nonzero((g_st["kept"] != r_st["kept"]) & ~topp_b)[0]
    assert kept_bad.size == 0, \
        f"kept-count mismatch rows {kept_bad[:10].tolist()}: gpu {g_st['kept'][kept_bad[:10]]} " \
        f"ref {r_st['kept'][kept_bad[:10]]}"
    drawn = (r_st["path"] == 4) & ~mism & ~topp_b
    if drawn.any():
        assert np.array_equal(g_st["u"][drawn], r_st["u"][drawn])
        rel_p = np.abs(g_st["prob"][drawn] - r_st["prob"][drawn]) / np.maximum(r_st["prob"][drawn],
                                                                              1e-300)
        rel_z = np.abs(g_st["z_kept"][drawn] - r_st["z_kept"][drawn]) / r_st["z_kept"][drawn]
        rep["max_prob_rel_err"] = float(rel_p.max())
        rep["max_zkept_rel_err"] = float(rel_z.max())
        assert rel_p.max() <= PROB_RTOL, f"prob rel err {rel_p.max()}"
        assert rel_z.max() <= PROB_RTOL, f"z_kept rel err {rel_z.max()}"
    margin = np.minimum(r_st["topp_margin"], r_st["cdf_margin"])
    loose = np.nonzero(mism & (margin > STRICT_BOUNDARY))[0]
    assert loose.size == 0, \
        f"mismatch rows {loose[:10].tolist()} with oracle margins {margin[loose[:10]]} > {STRICT_BOUNDARY}"
    rep["max_mismatch_margin"] = float(margin[mism].max()) if mism.any() else 0.0
    rep["sampled_mismatch"] = int(mism.sum())
    rep["topp_boundary_rows"] = int(topp_b.sum())
    rep["cdf_boundary_rows"] = int(cdf_b.sum())
    rep["boundary_mismatch"] = int((mism & boundary).sum())
    return rep
