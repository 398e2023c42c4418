// rng.h — the reference's per-sequence RNG, usable on host and device.
//
// nimbus-infer-rs `Rng` (src/sampler.rs:40-78): xoshiro256++ (Blackman &
// Vigna 2018) seeded through SplitMix64 (Steele, Lea & Flood 2014).  The
// reference advances its SplitMix counter once before the first output
// (sampler.rs:47 and 49), so the state is SplitMix64 outputs #2..#5.  The
// multipliers, shift and rotation amounts are the published constants of the
// two generators; they must be identical for the streams to agree.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define NIS_HD __host__ __device__ __forceinline__
#else
#define NIS_HD inline
#endif

namespace nis {

constexpr uint64_t kGoldenGamma = 0x9E3779B97F4A7C15ull;

NIS_HD uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

// Rng::new (sampler.rs:46-56)
NIS_HD void rng_seed(uint64_t seed, uint64_t s[4]) {
    uint64_t sm = seed + kGoldenGamma;
    for (int i = 0; i < 4; ++i) {
        sm += kGoldenGamma;
        uint64_t z = sm;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        s[i] = z ^ (z >> 31);
    }
}

// Rng::next_u64 (sampler.rs:58-72)
NIS_HD uint64_t rng_next_u64(uint64_t s[4]) {
    const uint64_t result = rotl64(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

// Rng::next_f64 (sampler.rs:75-77): top 53 bits times 2^-53, exact in f64.
NIS_HD double rng_next_f64(uint64_t s[4]) {
    return (double)(rng_next_u64(s) >> 11) * (1.0 / 9007199254740992.0);
}

}  // namespace nis
