"""Command-line surface of the GPU path, mirroring the reference's CLI.

  python -m nimbus_sampler bench-kernel   # cmd_bench_kernel (main.rs:372-445) on the GPU
  python -m nimbus_sampler bench-sampler  # the same JSON shape for sample() over a batch
  python -m nimbus_sampler generate ...   # cmd_generate's sampling flags (main.rs:136-189)
                                          # driving the device decode loop

generate takes the reference's options with their defaults and parsing
(--max-new-tokens 64, --temperature 0 = greedy, --top-k 0, --top-p 1.0,
--repetition-penalty 1.0, --seed unset = 0x5DEECE66D, --stream, --json;
nimbus_sampler/flags.py).  The model is outside this build, so each step's
logits come from the LM-head producer (nis_lm_head_logits) over a synthetic
f32 head and synthetic hidden states (--hidden H, --data-seed); the decode
step (nis_decode_step) samples on the device, and the ids are decoded on the
host with a byte-level BPE vocabulary (--vocab vocab.json, streamed with
--stream exactly as Engine::generate_stream does, engine.rs:296-316).
--batch B runs B sequences at once, sequence b seeded with seed + b.

bench-kernel builds the reference's synthetic 50257 x 768 head and hidden row
(main.rs:375-384: x[i] = ((i % 97) - 48) / 48, weights from i * 2654435761)
in the same formats — f32 rows, int8 biased bytes, int4 packed nibbles, no
scale (a scale of 1.0 per row here) — runs nis_lm_head_logits with one
hidden row, and prints the reference's keys (GFLOP/s, ms per pass, y[0] of
each format as checks) plus the published CPU figures for comparison.
"""
import argparse
import json
import sys

OUT, IN = 50257, 768
# README.md:45-51 of the reference, as quoted with the workload above
REFERENCE_GFLOPS = {"f32": 19.4, "int8": 22.5, "int4": 29.2}


def reference_kernel_inputs():
    """x, f32 weights, int8 codes, int4 bytes of main.rs:375-384."""
    import numpy as np
    x = ((np.arange(IN) % 97).astype(np.float32) - np.float32(48.0)) / np.float32(48.0)
    i = np.arange(OUT * IN, dtype=np.uint64)
    h = i * np.uint64(2654435761)
    w_f32 = ((h % np.uint64(2000)).astype(np.float32) - np.float32(1000.0)) / np.float32(10000.0)
    w_i8 = (h % np.uint64(256)).astype(np.uint8)
    j = np.arange(OUT * IN // 2, dtype=np.uint64)
    w_i4 = ((j * np.uint64(2654435761)) % np.uint64(256)).astype(np.uint8)
    return x.astype(np.float32), w_f32, w_i8, w_i4


def bench_kernel(steps=50, warmup=5, device=0):
    import numpy as np
    import torch
    from . import Sampler, W_F32, W_INT4, W_INT8
    x, w_f32, w_i8, w_i4 = reference_kernel_inputs()
    dev = torch.device("cuda", device)
    s = Sampler(device)
    xd = torch.from_numpy(np.ascontiguousarray(x.reshape(1, IN))).to(dev).contiguous()
    ones = torch.ones(OUT, dtype=torch.float32, device=dev)
    out = torch.empty((1, OUT), dtype=torch.float32, device=dev)
    res = {"kernel": f"dot {OUT}x{IN}"}
    checks, ms = [], {}
    for name, fmt, data in (("f32", W_F32, w_f32), ("int8", W_INT8, w_i8), ("int4", W_INT4, w_i4)):
        d = torch.from_numpy(data).to(dev)
        sc = None if fmt == W_F32 else ones
        for _ in range(warmup):
            s.lm_head_logits(xd, fmt, d, OUT, scales=sc, out=out)
        stream = torch.cuda.current_stream(dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            s.lm_head_logits(xd, fmt, d, OUT, scales=sc, out=out)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        ms[name] = e0.elapsed_time(e1) / steps
        checks.append(float(out[0, 0].item()))
    s.close()
    flops = 2.0 * OUT * IN
    for name in ("f32", "int8", "int4"):
        res[f"{name}_gflops"] = round(flops / (ms[name] * 1e-3) / 1e9, 1)
    for name in ("f32", "int8", "int4"):
        res[f"{name}_ms"] = round(ms[name], 4)
    res["checks"] = [round(c, 4) for c in checks]
    res["device"] = "MI355X (gfx950), one hidden row, mean of %d launches" % steps
    res["vs_reference_cpu"] = {k: round(res[f"{k}_gflops"] / v, 1) for k, v in REFERENCE_GFLOPS.items()}
    return res


def bench_sampler(steps=50, warmup=5, device=0, workload="headline"):
    import numpy as np
    import torch
    from . import SamplingParams, Sampler, rng_states, workloads
    w = workloads.WORKLOADS[workload]
    dev = torch.device("cuda", device)
    s = Sampler(device)
    x = torch.from_numpy(w.make(w.B)).to(dev)
    st = torch.from_numpy(rng_states(w.seeds).view(np.int64)).to(dev)
    params = SamplingParams(temperature=w.temperature, top_p=w.top_p)
    toks = torch.empty(w.B, dtype=torch.int32, device=dev)
    for _ in range(warmup):
        s.sample_batch(x, params, st, tokens=toks)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(torch.cuda.current_stream(dev))
    for _ in range(steps):
        s.sample_batch(x, params, st, tokens=toks)
    e1.record(torch.cuda.current_stream(dev))
    torch.cuda.synchronize(dev)
    msv = e0.elapsed_time(e1) / steps
    first = toks[:4].cpu().tolist()
    s.close()
    return {"kernel": f"sample {w.B}x{w.V} T={w.temperature} top-p={w.top_p}",
            "rows_per_s": round(w.B / (msv * 1e-3), 1), "ms": round(msv, 4),
            "logits_gbs": round(w.B * w.V * 4 / (msv * 1e-3) / 1e9, 1), "checks": first,
            "note": "one batch re-read by every launch (it can stay in the 256 MB cache); "
                    "bench.py rotates 8 batches for the HBM figure"}


def generate(args, out=None, keep_logits=False):
    """cmd_generate (main.rs:136-189) with the model step replaced by the
    synthetic LM head: parse the reference's flags, run the device decode
    loop, decode the ids on the host.  Returns a dict with the params, the
    seed, each sequence's ids and text (and the per-step logits on request)."""
    import time
    import numpy as np
    import torch
    from . import Sampler, W_F32, Rng
    from .flags import generate_params
    from .stream import BatchStreams, TokenBytes
    params, seed, flags = generate_params(list(args))
    vocab_path = flags.get("vocab")
    table = TokenBytes.from_file(vocab_path) if vocab_path else None
    V = len(table) if table is not None else flags.usize_of("vocab-size", 50257)
    H = flags.usize_of("hidden", 64)
    B = max(flags.usize_of("batch", 1), 1)
    dseed = flags.usize_of("data-seed", 0)
    device = flags.usize_of("device", 0)
    n_new = params.max_new_tokens
    dev = torch.device("cuda", device)
    rnd = np.random.Generator(np.random.PCG64(dseed))
    # a head whose logits spread like a trained model's (std ~3)
    w = (rnd.standard_normal((V, H)) * (3.0 / np.sqrt(H))).astype(np.float32)
    wd = torch.from_numpy(w.reshape(-1)).to(dev)
    s = Sampler(device)
    cap = max(n_new, 1)
    states = torch.from_numpy(np.array([Rng(seed + b).state() for b in range(B)],
                                       dtype=np.uint64).view(np.int64)).to(dev)
    gen_ids = torch.zeros((B, cap), dtype=torch.int32, device=dev)
    gen_len = torch.zeros(B, dtype=torch.int32, device=dev)
    max_new = torch.full((B,), n_new, dtype=torch.int32, device=dev)
    done = torch.full((B,), 1 if n_new <= 0 else 0, dtype=torch.uint8, device=dev)
    tokens = torch.zeros(B, dtype=torch.int32, device=dev)
    logits = torch.empty((B, V), dtype=torch.float32, device=dev)
    streams = BatchStreams(table, B) if table is not None else None
    ids = [[] for _ in range(B)]
    kept_logits = []
    t0 = time.perf_counter()
    for step in range(n_new):
        live = done.cpu().numpy() == 0
        if not live.any():
            break
        hid = torch.from_numpy(rnd.standard_normal((B, H)).astype(np.float32)).to(dev)
        s.lm_head_logits(hid, W_F32, wd, V, out=logits)
        if keep_logits:
            kept_logits.append(logits.cpu().numpy().copy())
        s.decode_step(logits, params, states, gen_ids, gen_len, max_new, done, tokens=tokens)
        tok = tokens.cpu().numpy().view(np.uint32)
        for b in range(B):
            if live[b]:
                ids[b].append(int(tok[b]))
        if streams is not None:
            deltas = streams.push_step(tok, live)
            if flags.has("stream") and out is not None and deltas[0]:
                out.write(deltas[0])
                out.flush()
    if streams is not None:
        tail = streams.flush()
        if flags.has("stream") and out is not None and tail[0]:
            out.write(tail[0])
    dt = time.perf_counter() - t0
    s.close()
    texts = streams.text if streams is not None else [str(x) for x in ids]
    res = {"params": params, "seed": seed, "ids": ids, "texts": texts, "seconds": dt,
           "flags": flags}
    if keep_logits:
        res["logits"] = kept_logits
    return res


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    if argv and argv[0] == "generate":
        if "--help" in argv[1:] or "-h" in argv[1:]:
            print(__doc__)
            return 0
        res = generate(argv[1:], out=sys.stdout)
        flags = res["flags"]
        n = len(res["ids"][0])
        if flags.has("stream"):
            print()
        elif flags.has("json"):
            print(json.dumps({"generated_ids": res["ids"][0], "text": res["texts"][0],
                              "seed": res["seed"]}))
        else:
            print(res["texts"][0])
        print(f"[{n} tokens in {res['seconds']:.2f}s = {n / max(res['seconds'], 1e-9):.1f} tok/s]",
              file=sys.stderr)
        return 0
    ap = argparse.ArgumentParser(prog="python -m nimbus_sampler")
    sub = ap.add_subparsers(dest="cmd", required=True)
    for name in ("bench-kernel", "bench-sampler"):
        p = sub.add_parser(name)
        p.add_argument("--steps", type=int, default=50)
        p.add_argument("--warmup", type=int, default=5)
        p.add_argument("--device", type=int, default=0)
    sub.add_parser("generate", help="sampling flags of the reference's generate, on the "
                                    "device decode loop (see the module docstring)")
    args = ap.parse_args(argv)
    if args.cmd == "bench-kernel":
        print(json.dumps(bench_kernel(args.steps, args.warmup, args.device)))
    else:
        print(json.dumps(bench_sampler(args.steps, args.warmup, args.device)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
