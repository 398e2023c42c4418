#!/usr/bin/env python3
"""Benchmark of the MI355X sampler on the headline workload.

Metric: sampled rows/s + HBM GB/s (% of peak) for
B=256 x V=50257 fp32 logits, T=0.8, top-p=0.9.  A step is one
nis_sample_batch() launch over one [256, 50257] batch that is already
resident in HBM.  Eight distinct input batches (412 MB) are rotated so
reads cannot be served from the 256 MB Infinity Cache.

JSON line fields beyond the driver contract:
  roofline      dominant kernel: algorithmic bytes per launch
                B*(4V + 68) (logits once, token, 32 B RNG state in + out)
                over its mean launch duration: HIP events bracketing the
                timed hipGraph replays on the launch stream, divided by the
                number of launches; traffic from the committed rocprofv3
                --pmc summary when present.
  cpu_baseline  the CPU oracle (a C restatement of sampler.rs) over the
                same 256 rows with the threads.rs fork-join, median of 5
                batches after one warm-up.
  parity        first timed batch vs the oracle (greedy and sampled).
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nimbus-infer-rs_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/s + HBM GB/s (% peak), B=256 x V=50257 fp32, T=0.8 top-p=0.9"
GRAPH_MAX = 200          # launches per captured hipGraph in the timed region
RESIDENT_MAX_V = 53245   # kRMaxV: the largest row one 1024-lane workgroup holds in registers
LONG_SPARSE_MAX_V = 262141  # kLSMaxV: the longest row the single-read long kernel takes
SPARSE_MAX_V = 53245     # kSMaxV


def routed_kernel(V, temperature, top_k, top_p, penalty, history=False):
    """The kernel nis_sample_batch launches for these parameters (launch_rows
    in capi.hip)."""
    res_shape = 256 <= V <= RESIDENT_MAX_V
    no_topk = top_k == 0 or top_k >= V
    if V > RESIDENT_MAX_V and temperature <= 0.0:
        return "sample_rows_long_kernel<greedy>"
    if (RESIDENT_MAX_V < V <= LONG_SPARSE_MAX_V and 0.0 < top_p < 0.95 and (top_k == 0 or top_k >= V)
            and (penalty == 1.0 or not history)):
        return "sample_rows_long_sparse_kernel"
    if V > RESIDENT_MAX_V and (top_k == 0 or top_k >= V) and (penalty == 1.0 or not history):
        return "sample_rows_long_kernel<all>" if top_p >= 1.0 else "sample_rows_long_kernel<top-p>"
    pen = penalty != 1.0 and history
    if res_shape and temperature <= 0.0:
        return "sample_rows_resident_kernel<greedy-pen>" if pen else "sample_rows_resident_kernel<greedy>"
    if res_shape and temperature > 0.0 and no_topk and top_p >= 1.0:
        return "sample_rows_resident_kernel<all-pen>" if pen else "sample_rows_resident_kernel<all>"
    if res_shape and temperature > 0.0 and no_topk and 0.95 <= top_p < 1.0 \
            and (penalty == 1.0 or not history):
        return "sample_rows_dense_kernel"
    if 256 <= V <= SPARSE_MAX_V and temperature > 0.0 and top_p > 0.0 and not no_topk \
            and not (penalty != 1.0 and history):
        return "sample_rows_sparse_topk_kernel"
    if 256 <= V <= SPARSE_MAX_V and temperature > 0.0 and 0.0 < top_p < 0.95 and no_topk:
        if penalty != 1.0 and history:
            return "sample_rows_sparse_pen_kernel"
        return "sample_rows_sparse_kernel"
    return "sample_rows_kernel"


def host_cpu():
    """Host CPU model and the logical cores this process may run on."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "nproc": len(os.sched_getaffinity(0)),
            "os_cpu_count": os.cpu_count()}


def reference_worker_count():
    """threads.rs:12-26 worker_count(): NIMBUS_THREADS when it parses to a
    positive integer, else every logical core the process may run on
    (std::thread::available_parallelism follows the affinity mask)."""
    v = os.environ.get("NIMBUS_THREADS")
    if v is not None:
        try:
            n = int(v)
            if n > 0:
                return n
        except ValueError:
            pass
    return len(os.sched_getaffinity(0))


def replay_exact(graph_full, graph_tail, G, K):
    """K launches: K // G replays of the G-launch graph, then the K % G tail."""
    for _ in range(K // G):
        graph_full.replay()
    if K % G:
        graph_tail.replay()


def capture(fn, n):
    """A hipGraph of fn(0), ..., fn(n-1) captured on a side stream."""
    import torch
    if n == 0:
        return None
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            for i in range(n):
                fn(i)
    torch.cuda.current_stream().wait_stream(cap)
    return graph


def read_traffic(workload, kernel):
    """HBM bytes per launch of this workload's kernel from the committed
    rocprofv3 --pmc summary profiles/*traffic*<workload>*.txt (FETCH_SIZE +
    WRITE_SIZE per dispatch, scaled by a plain copy's reading); None when no
    summary for this kernel exists.  Returns (bytes, source file)."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None, None
    base = kernel.split("<")[0]
    for fn in sorted(os.listdir(pdir)):
        if "traffic" in fn and fn.endswith(f"_{workload}.txt"):
            with open(os.path.join(pdir, fn)) as f:
                text = f.read()
            k = re.search(r"^kernel:\s*(\S+)", text, re.M)
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
            if m and (k is None or k.group(1).split("<")[0] == base):
                return float(m.group(1)), f"profiles/{fn}"
    return None, None


def bench_decode(args, w, sampler, params, bufs, states, tokens):
    """Decode steps (engine.rs:279-287 on the device): one nis_decode_step per
    rotated batch, sequences never finishing (budget and history capacity
    above the steps of a replay, which starts by clearing lengths and flags)."""
    import torch
    B, V = w.B, w.V
    dev = tokens.device
    H = args.history
    cap = 64 + H
    # the first H ids of every history: random tokens already generated
    gen_ids = torch.randint(0, V, (B, cap), generator=torch.Generator().manual_seed(3),
                            dtype=torch.int32).to(dev)
    gen_len = torch.zeros(B, dtype=torch.int32, device=dev)
    max_new = torch.full((B,), cap, dtype=torch.int32, device=dev)
    done = torch.zeros(B, dtype=torch.uint8, device=dev)
    G = len(bufs)

    def block(n):
        gen_len.fill_(H)
        done.zero_()
        for i in range(n):
            sampler.decode_step(bufs[i], params, states, gen_ids, gen_len, max_new, done,
                                tokens=tokens)

    for i in range(args.warmup):
        if i % G == 0:
            gen_len.fill_(H)
            done.zero_()
        sampler.decode_step(bufs[i % G], params, states, gen_ids, gen_len, max_new, done,
                            tokens=tokens)
    torch.cuda.synchronize()
    K = max(1, args.steps)
    g_full = capture(lambda _: block(G), 1)
    g_tail = capture(lambda _: block(K % G), 1) if K % G else None
    for _ in range(2):
        g_full.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    replay_exact(g_full, g_tail, G, K)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / K
    assert int(gen_len[0].item()) == H + (K % G or G) and int(done.sum().item()) == 0
    alg_bytes = B * (4 * V + 68) + B * (4 + 4 + 1)  # logits, RNG, token + history, length, flag
    if params.repetition_penalty != 1.0:
        alg_bytes += B * 4 * H  # the histories read as penalty lists (at least H ids each)
    print(json.dumps({
        "metric": f"decode steps: tokens/s, B={B} sequences x V={V} fp32, "
                  f"T={params.temperature} top-p={params.top_p} "
                  f"repetition-penalty={params.repetition_penalty}",
        "value": B / (us * 1e-6), "unit": "tokens/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "us_per_step": us, "higher_is_better": True,
        "data": "synthetic logits of the workload, 8 rotated batches resident in HBM",
        "config": {"workload": args.workload, "B": B, "V": V, "history_cap": cap,
                   "history_at_start": H, "repetition_penalty": params.repetition_penalty,
                   "launch": f"hipGraph replays of up to {G} nis_decode_step calls after "
                             "clearing the lengths and flags"},
        "roofline": {"bound": "hbm", "achieved": alg_bytes / (us * 1e-6) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": alg_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS},
    }))

def bench_floor(args, w, sampler, bufs):
    """The stream floor (nis_stream_floor) on the workload's batches, timed
    exactly as the sampler is: the same graph replays and events."""
    import torch
    B, V = w.B, w.V
    out = torch.empty((B, 2), dtype=torch.float32, device=bufs[0].device)
    nb = len(bufs)
    S = args.split
    part = torch.empty((max(S, 1) * B * 4, 4), dtype=torch.float32, device=bufs[0].device)

    def launch(i):
        if S:
            sampler.stream_floor_split(bufs[i % nb], w.temperature, S, out=out, part=part)
        else:
            sampler.stream_floor(bufs[i % nb], w.temperature, out=out)

    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    K = max(1, args.steps)
    G = min(GRAPH_MAX, K)
    g_full = capture(launch, G)
    g_tail = capture(launch, K % G)
    for _ in range(2):
        g_full.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    replay_exact(g_full, g_tail, G, K)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / K
    alg_bytes = B * 4 * V
    what = (f"each row split over {S} workgroups of 256 lanes, partials merged by a second launch"
            if S else "the sparse kernel's layout")
    print(json.dumps({
        "metric": f"stream floor: rows/s + HBM GB/s (% peak), B={B} x V={V} fp32 read with "
                  f"{what} (max and exp-sum only, nothing sampled)",
        "value": B / (us * 1e-6), "unit": "rows/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "us_per_step": us, "higher_is_better": True,
        "data": "synthetic logits of the workload, 8 rotated batches resident in HBM",
        "config": {"workload": args.workload, "B": B, "V": V,
                   "launch": f"hipGraph replays of up to {G} "
                             f"{'nis_stream_floor_split calls (2 launches each)' if S else 'nis_stream_floor launches'}"},
        "roofline": {"bound": "hbm", "achieved": alg_bytes / (us * 1e-6) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": alg_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                     "kernel": "split_floor_part_kernel + split_floor_merge_kernel" if S
                     else "stream_floor_kernel", "launch_interval_us": us,
                     "alg_bytes_per_launch": alg_bytes},
    }))


MFMA_F32_PEAK_TFLOPS = 157.3


def bench_lm_head(args):
    """The logits producer (model.rs:317-325) on its own: B last-hidden rows
    against a [V, H] head in the chosen weight format, K launches timed with
    events on the stream the kernel runs on."""
    import time
    import numpy as np
    import torch
    import nimbus_sampler as ns
    from nimbus_sampler import workloads

    w = workloads.WORKLOADS[args.workload]
    B, V, H = args.lm_b, w.V, args.lm_h
    fmt = {"f32": ns.W_F32, "int8": ns.W_INT8, "int4": ns.W_INT4}[args.lm_head]
    group = args.lm_group if fmt != ns.W_F32 else 0
    dev = torch.device("cuda:0")
    rnd = np.random.default_rng(0)
    x = torch.from_numpy(rnd.standard_normal((B, H)).astype(np.float32)).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    groups = H // group if group else 1
    if fmt == ns.W_F32:
        data = torch.randn((V, H), generator=g, device=dev) * 0.05
        wbytes = V * H * 4
    else:
        nbytes = V * H if fmt == ns.W_INT8 else (V * H + 1) // 2
        data = torch.randint(0, 256, (nbytes,), generator=g, device=dev, dtype=torch.int32) \
            .to(torch.uint8)
        wbytes = nbytes + V * groups * 4
    scales = (torch.rand((V * groups,), generator=g, device=dev) * 0.02 + 0.005) \
        if fmt != ns.W_F32 else None
    out = torch.empty((B, V), dtype=torch.float32, device=dev)
    sampler = ns.Sampler(0)
    # distinct copies of the head, rotated launch by launch, so the working
    # set (>= 768 MiB) is three times the 256 MiB MALL and every launch
    # reads its head from HBM
    ncopy = max(2, -(-(768 << 20) // wbytes))
    heads = [(data, scales)] + [(data.clone(), scales.clone() if scales is not None else None)
                                for _ in range(ncopy - 1)]

    greedy = args.greedy and B == 1
    tok = torch.empty(1, dtype=torch.int32, device=dev)

    def run(i):
        d, sc = heads[i % ncopy]
        if greedy:
            sampler.lm_head_greedy(x[0], fmt, d, V, scales=sc, group_size=group, token=tok)
        else:
            sampler.lm_head_logits(x, fmt, d, V, scales=sc, group_size=group, out=out)

    def run_split(i):  # the two-call form the fused one replaces
        d, sc = heads[i % ncopy]
        sampler.lm_head_logits(x, fmt, d, V, scales=sc, group_size=group, out=out)
        sampler.argmax_batch(out, tokens=tok)

    # --sample (B = 1): the decode step's sampled form, GEMV then
    # nis_sample_batch on the logits it just wrote (T 0.8, top-p 0.9).  The
    # hidden row is rescaled so the logits have c1's spread (standard
    # deviation 3): the random heads' own logits are far narrower or wider,
    # and a nucleus past the sparse kernel's lists would time the general
    # path instead of the sampler the decode loop runs on real logits.
    sparams = ns.SamplingParams(temperature=0.8, top_p=0.9)
    sstate = torch.from_numpy(ns.rng_states([7]).view(np.int64)).to(dev)
    xs = x
    if args.sample and B == 1:
        d0, sc0 = heads[0]
        sampler.lm_head_logits(x, fmt, d0, V, scales=sc0, group_size=group, out=out)
        torch.cuda.synchronize()
        xs = x * float(3.0 / max(float(out[0].std()), 1e-30))

    def run_sample(i):
        d, sc = heads[i % ncopy]
        sampler.lm_head_logits(xs, fmt, d, V, scales=sc, group_size=group, out=out)
        sampler.sample_batch(out, sparams, sstate, tokens=tok)

    def run_sample_only(i):
        sampler.sample_batch(out, sparams, sstate, tokens=tok)

    for i in range(args.warmup):
        run(i)
    torch.cuda.synchronize()
    K = args.steps
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(K):
        run(i)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / K
    split_us = None
    sample_us = sample_only_us = None
    if args.sample and B == 1:
        for fn in (run_sample, run_sample_only):
            for i in range(args.warmup):
                fn(i)
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(K):
                fn(i)
            e1.record(stream)
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) * 1e3 / K
            if fn is run_sample:
                sample_us = t
            else:
                sample_only_us = t  # the sampler alone on the same (hot) logits
    if greedy:
        for i in range(args.warmup):
            run_split(i)
        e0.record(stream)
        for i in range(K):
            run_split(i)
        e1.record(stream)
        torch.cuda.synchronize()
        split_us = e0.elapsed_time(e1) * 1e3 / K
    flops = 2.0 * B * V * H
    alg_bytes = wbytes + B * H * 4 + (4 if greedy else B * V * 4)
    t_mfma = flops / (MFMA_F32_PEAK_TFLOPS * 1e12)
    t_hbm = alg_bytes / (HBM_PEAK_GBS * 1e9)
    if t_mfma >= t_hbm:
        roof = {"bound": "mfma", "achieved": flops / (us * 1e-6) / 1e12,
                "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": alg_bytes / (us * 1e-6) / 1e9,
                "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = None
    cpu = None
    if not args.no_cpu_baseline:
        # the oracle's exact-sum restatement on a bounded sample of rows; its
        # output also checks the GPU's rows of the last launch (copy K-1)
        from oracle import lm_head_oracle as lh
        d, sc_t = heads[(K - 1) % ncopy]
        hd = d.cpu().numpy().reshape(-1)
        sc = sc_t.cpu().numpy() if sc_t is not None else None
        nb = min(B, 8)
        xs = x[:nb].cpu().numpy()
        t0 = time.perf_counter()
        exact, absum = lh.lm_head_logits(xs, fmt, hd, sc, V, H, group or None)
        dt = time.perf_counter() - t0
        got = out[:nb].cpu().numpy().astype(np.float64)
        bound = lh.f32_bound(absum, H, groups)
        err = float((np.abs(got - exact) / np.maximum(bound, 1e-300)).max())
        assert err <= 1.0, f"LM-head output outside the f32 error bound: {err}"
        cpu = {"value": nb / dt, "unit": "hidden rows/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{nb} hidden rows through oracle/lm_head_oracle.py, an f64 numpy "
                         "restatement of quant.rs/simd.rs (not the reference's f32 SIMD loop)",
               "check": f"GPU rows within {err:.3f} of the f32 summation error bound"}
    print(json.dumps({
        "metric": (f"LM head + greedy token (fused): decode steps/s, H={H} -> V={V}, "
                   f"{args.lm_head} weights" if greedy else
                   f"LM-head logits: hidden rows/s, B={B} x H={H} -> V={V}, {args.lm_head} weights")
                  + (f" (groups of {group})" if group else ""),
        "value": B / (us * 1e-6), "unit": "hidden rows/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": us / 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": f"synthetic hidden rows and random weights, {ncopy} head copies rotated "
                "(working set past the 256 MiB MALL)",
        "config": {"workload": f"lm_head_{args.lm_head}", "B": B, "H": H, "V": V,
                   "group_size": group, "alg_bytes": alg_bytes, "flops": flops,
                   "head_copies": ncopy,
                   "split_logits_then_argmax_us": split_us,
                   "logits_then_sample_us": sample_us,
                   "sample_on_hot_logits_us": sample_only_us},
        "roofline": roof, "cpu_baseline": cpu,
    }))
    sampler.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="headline")
    ap.add_argument("--buffers", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="oracle worker threads (0: threads.rs worker_count(): NIMBUS_THREADS, "
                         "else every logical core this process may run on)")
    ap.add_argument("--decode", action="store_true",
                    help="time nis_decode_step (sample + on-device history / stop / budget "
                         "update) on the workload instead, and print that line")
    ap.add_argument("--top-k", type=int, default=0,
                    help="top-k of every row (sampler.rs:103-116) on top of the workload's "
                         "temperature and top-p; the line's metric then names it")
    ap.add_argument("--penalty", type=float, default=1.0,
                    help="repetition penalty of --decode (sampler.rs:83-101; the histories "
                         "are the penalty lists)")
    ap.add_argument("--temperature", type=float, default=None,
                    help="temperature of --decode instead of the workload's (0: greedy)")
    ap.add_argument("--top-p", type=float, default=None,
                    help="top-p of --decode instead of the workload's (1: off)")
    ap.add_argument("--history", type=int, default=0,
                    help="ids already in every history when a --decode replay starts")
    ap.add_argument("--lm-head", choices=("f32", "int8", "int4"), default=None,
                    help="time the LM-head logits producer with these weights instead")
    ap.add_argument("--lm-b", type=int, default=256, help="hidden rows for --lm-head")
    ap.add_argument("--greedy", action="store_true",
                    help="with --lm-head and --lm-b 1: time nis_lm_head_greedy (GEMV with the "
                         "greedy token in its epilogue) and, beside it, nis_lm_head_logits + "
                         "nis_argmax_batch")
    ap.add_argument("--sample", action="store_true",
                    help="with --lm-head and --lm-b 1: also time nis_lm_head_logits followed by "
                         "nis_sample_batch (T 0.8, top-p 0.9) on the logits it wrote")
    ap.add_argument("--lm-h", type=int, default=768, help="hidden size for --lm-head")
    ap.add_argument("--lm-group", type=int, default=0, help="group size for quantized --lm-head")
    ap.add_argument("--floor", action="store_true",
                    help="time nis_stream_floor instead: the sparse kernel's layout and load "
                         "pipeline computing only each row's max and exp-sum (the bandwidth "
                         "ceiling the sampler's roofline fraction is measured against)")
    ap.add_argument("--split", type=int, default=0, metavar="S",
                    help="with --floor: time nis_stream_floor_split, each row read by S "
                         "workgroups and merged by a second launch (the least a sampler that "
                         "splits rows pays per merge)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 4 plain device copies of MIB MiB (reads MIB, writes MIB) "
                         "to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE, then exit")
    args = ap.parse_args()

    if args.calibrate_copy:
        import torch
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": 4 * n, "launches": 4}))
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this sampler build runs on one GPU only (rows are independent; "
              "row sharding across GPUs is not built). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.lm_head:
        bench_lm_head(args)
        return

    import numpy as np
    import torch
    import nimbus_sampler as ns
    from nimbus_sampler import workloads

    w = workloads.WORKLOADS[args.workload]
    B, V = w.B, w.V
    dev = torch.device("cuda:0")
    sampler = ns.Sampler(0)
    temp = args.temperature if (args.decode and args.temperature is not None) else w.temperature
    top_p = args.top_p if (args.decode and args.top_p is not None) else w.top_p
    params = ns.SamplingParams(temperature=temp, top_p=top_p, top_k=args.top_k,
                               repetition_penalty=args.penalty if args.decode else 1.0)

    host0 = w.make(B)
    # distinct batches of the same distribution: rows permuted, columns rolled
    bufs = [torch.from_numpy(workloads.rotation(host0, i)).to(dev) for i in range(args.buffers)]
    states = torch.from_numpy(ns.rng_states(w.seeds).view(np.int64)).to(dev)
    tokens = torch.empty(B, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    if args.decode:
        bench_decode(args, w, sampler, params, bufs, states, tokens)
        sampler.close()
        return
    if args.floor:
        bench_floor(args, w, sampler, bufs)
        sampler.close()
        return

    # parity of one batch against the oracle (state copy so the timed run is unaffected)
    parity = None
    try:
        from oracle import oracle
    except Exception:
        oracle = None
    if oracle is not None:
        st_copy = states.clone()
        stats = torch.zeros((B, 64), dtype=torch.uint8, device=dev)
        sampler.sample_batch(bufs[0], params, st_copy, tokens=tokens, stats=stats)
        g = sampler.argmax_batch(bufs[0])
        torch.cuda.synchronize()
        ref_states = oracle.rng_states(w.seeds)
        rt, rs, _ = oracle.sample_batch(host0, V, oracle.make_params(w.temperature, w.top_p, args.top_k),
                                        ref_states)
        gt, _, _ = oracle.sample_batch(host0, V, oracle.make_params(0.0), oracle.rng_states(w.seeds))
        got = tokens.cpu().numpy().astype(np.uint32)
        boundary = (rs["topp_margin"] <= 1e-6) | (rs["cdf_margin"] <= 1e-6)
        mism = got != rt
        margin = np.minimum(rs["topp_margin"], rs["cdf_margin"])
        parity = {
            "greedy_mismatch": int((g.cpu().numpy().astype(np.uint32) != gt).sum()),
            "sampled_mismatch_outside_boundary": int((mism & ~boundary).sum()),
            "boundary_rows": int(boundary.sum()),
            # rows whose sampled id differs from the oracle's, all of them on an
            # oracle boundary, and the largest oracle margin among them
            "boundary_mismatch": int((mism & boundary).sum()),
            "max_mismatch_margin": float(margin[mism].max()) if mism.any() else 0.0,
            "rng_state_match": bool(np.array_equal(st_copy.cpu().numpy().view(np.uint64), ref_states)),
        }

    for i in range(args.warmup):
        sampler.sample_batch(bufs[i % len(bufs)], params, states, tokens=tokens)
    torch.cuda.synchronize()

    # Timed region: hipGraph replays of launches over the rotated buffers
    # (launch i reads buffer i mod 8), so the GPU is not waiting on Python
    # between launches.  A graph holds up to GRAPH_MAX launches: each replay
    # boundary costs about 5 us, so short graphs would add ~0.7 us per launch.
    # HIP events bracket the whole region on the stream the launches run on;
    # the launch interval is their elapsed time over the number of launches.
    G = min(GRAPH_MAX, max(1, args.steps))
    K = max(1, args.steps)
    nb = len(bufs)

    def launch(i):
        sampler.sample_batch(bufs[i % nb], params, states, tokens=tokens)

    g_full = capture(launch, G)
    g_tail = capture(launch, K % G)
    for _ in range(2):  # warm replays
        g_full.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    replay_exact(g_full, g_tail, G, K)
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall = t1 - t0
    mean_ms = e0.elapsed_time(e1) / K

    # eager rate through the Python binding (one ctypes call per batch), for reference
    torch.cuda.synchronize()
    te0 = time.perf_counter()
    for i in range(min(K, 64)):
        sampler.sample_batch(bufs[i % nb], params, states, tokens=tokens)
    torch.cuda.synchronize()
    eager_rows_s = B * min(K, 64) / (time.perf_counter() - te0)

    alg_bytes = B * (4 * V + 68)
    achieved = alg_bytes / (mean_ms * 1e-3) / 1e9
    kernel = routed_kernel(V, w.temperature, args.top_k, w.top_p, 1.0)
    traffic, traffic_src = read_traffic(
        args.workload if not args.top_k else f"{args.workload}_topk{args.top_k}", kernel)

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle
        nthreads = args.cpu_threads or reference_worker_count()
        p = oracle.make_params(w.temperature, w.top_p, args.top_k)
        times = []
        for rep in range(6):
            st = oracle.rng_states(w.seeds)
            c0 = time.perf_counter()
            _, _, used = oracle.sample_batch(host0, V, p, st, n_threads=nthreads)
            times.append(time.perf_counter() - c0)
        times = sorted(times[1:])
        med = times[len(times) // 2]
        cpu = {"value": B / med, "unit": "rows/s", "cores": used, "kind": "port",
               "sample": f"C restatement of sampler.rs over the same {B}x{V} batch, "
                         f"threads.rs fork-join on {used} threads (worker_count(): "
                         f"NIMBUS_THREADS, else every logical core), median of 5 batches "
                         f"after 1 warm-up",
               "gbs": alg_bytes / med / 1e9, "host": host_cpu()}

    metric = METRIC if (args.workload == "headline" and not args.top_k) else \
        (f"sampled rows/s + HBM GB/s (% peak), B={B} x V={V} fp32, T={w.temperature} "
         f"top-p={w.top_p}" + (f" top-k={args.top_k}" if args.top_k else ""))
    out = {
        "metric": metric,
        "value": B * K / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / K,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": f"synthetic: {w.description}; 8 rotated batches resident in HBM",
        "config": {"workload": args.workload, "B": B, "V": V, "temperature": w.temperature,
                   "top_p": w.top_p, "top_k": args.top_k, "ld": V, "parallelism": "1 GPU",
                   "launch": f"hipGraph replays: {K // G} x {G} + {K % G} nis_sample_batch "
                             f"launches over {nb} rotated batches",
                   "eager_rows_per_s": eager_rows_s},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": (f"{traffic_src}: rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE "
                                        "per dispatch, scaled by a plain copy's reading")
                     if traffic_src else None,
                     "kernel": kernel,
                     # HIP-event interval over the timed replays / launches: the
                     # kernel's duration plus the gap between graph nodes (the
                     # rocprofv3 kernel durations are in profiles/)
                     "launch_interval_us": mean_ms * 1e3,
                     "alg_bytes_per_launch": alg_bytes},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(out))
    sampler.close()


if __name__ == "__main__":
    main()
