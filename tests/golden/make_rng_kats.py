"""Write tests/golden/rng_kats.json: known answers of the reference RNG.

An independent pure-Python (big-int) restatement of nimbus-infer-rs
`Rng::new` / `next_u64` / `next_f64` (src/sampler.rs:46-77), written from
the published SplitMix64 and xoshiro256++ definitions with the reference's
seeding quirk (the SplitMix counter is advanced once before the first draw,
sampler.rs:47 and 49).  It shares no code with the C oracle or the HIP
kernels, so agreement of all three pins the RNG.

Run:  python tests/golden/make_rng_kats.py
"""
import json
import os

M64 = (1 << 64) - 1


def splitmix64_stream(seed, n):
    """Plain SplitMix64: n outputs starting from counter `seed`."""
    out, sm = [], seed & M64
    for _ in range(n):
        sm = (sm + 0x9E3779B97F4A7C15) & M64
        z = sm
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out.append(z ^ (z >> 31))
    return out


def rng_new(seed):
    # the reference's state is SplitMix64 outputs #2..#5
    return splitmix64_stream(seed, 5)[1:]


def rotl(x, k):
    return ((x << k) | (x >> (64 - k))) & M64


def next_u64(s):
    result = (rotl((s[0] + s[3]) & M64, 23) + s[0]) & M64
    t = (s[1] << 17) & M64
    s[2] ^= s[0]
    s[3] ^= s[1]
    s[1] ^= s[2]
    s[0] ^= s[3]
    s[2] ^= t
    s[3] = rotl(s[3], 45)
    return result


def main():
    seeds = [0, 1, 7, 42, 43, 63, 1000, 2023, 0x5DEECE66D, M64, 1 << 63]
    kats = []
    for seed in seeds:
        s = rng_new(seed)
        state0 = list(s)
        u64s = [next_u64(s) for _ in range(8)]
        s2 = rng_new(seed)
        f64 = (next_u64(s2) >> 11) / float(1 << 53)
        kats.append({
            "seed": str(seed),
            "state": [str(v) for v in state0],
            "next_u64": [str(v) for v in u64s],
            "first_f64": repr(f64),
            "state_after_8": [str(v) for v in s],
        })
    doc = {
        "generator": "tests/golden/make_rng_kats.py (Python big-int restatement)",
        "splitmix64_seed0_first5": [str(v) for v in splitmix64_stream(0, 5)],
        "kats": kats,
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rng_kats.json")
    with open(path, "w") as f:
        json.dump(doc, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
