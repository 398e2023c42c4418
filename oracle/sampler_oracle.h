/*
 * sampler_oracle.h — CPU restatement of nimbus-infer-rs `src/sampler.rs`.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker that the HIP sampler is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it and has
 * no CPU fallback.
 *
 * Every function follows the reference operation by operation in IEEE f64
 * (no fast-math, no FMA contraction, glibc `exp`), citing the lines of
 * /root/reference/src/sampler.rs it restates.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   oracle_rng_*                  published SplitMix64(0) stream, big-integer
 *                                 KATs (tests/golden/rng_kats.json), GF(2)
 *                                 linearity, sampler.rs:230-239
 *   oracle_apply_repetition_penalty  sampler.rs:251-257, brute force
 *   oracle_top_k_filter           sampler.rs:241-249, brute force on tiny rows
 *   oracle_top_p_filter           sampler.rs:259-266 (p = 0), exact-rational
 *                                 brute force of the keep rule on tiny rows,
 *                                 prefix / tie-group invariants
 *   oracle_sample                 sampler.rs:223-228, exact-rational inverse
 *                                 CDF on 4000 tiny rows, special rows
 *   oracle_sample_batch           equals sequential oracle_sample
 * Parity unpinned (no reference build or value fixture exists here): the
 * bit pattern of `exp` (Rust's f64::exp lowers to the platform libm, glibc
 * here) and the last-bit rounding of the sequential sorted-order and CDF
 * sums at exact boundaries; the GPU tests treat rows within 1e-6 of such a
 * boundary as boundary rows and count them.
 */
#ifndef NIMBUS_SAMPLER_ORACLE_H
#define NIMBUS_SAMPLER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same fields and f32 types as SamplingParams' sampling knobs
 * (sampler.rs:7-15); laid out like `nis_params` in include/nimbus_sampler.h. */
typedef struct oracle_params {
    float temperature;
    float top_p;
    float repetition_penalty;
    uint32_t _pad;
    uint64_t top_k;
} oracle_params;

/* Which branch of `sample()` produced the token. */
enum {
    ORACLE_PATH_GREEDY = 1,       /* sampler.rs:172-181 */
    ORACLE_PATH_NONFINITE_MAX = 2,/* sampler.rs:192-200 */
    ORACLE_PATH_BAD_TOTAL = 3,    /* sampler.rs:206-208 */
    ORACLE_PATH_DRAW = 4,         /* sampler.rs:209-214 */
    ORACLE_PATH_FALLTHROUGH = 5   /* sampler.rs:216 */
};

/* Diagnostics of one `sample()` call, used to classify boundary rows. */
typedef struct oracle_stats {
    double max_w;        /* max of the filtered, temperature-scaled logits (sampler.rs:191) */
    double z_kept;       /* `total` (sampler.rs:201-205) */
    double z_sorted;     /* top-p `sum` in sorted order (sampler.rs:143), 0 if top-p inactive */
    double u;            /* next_f64() drawn at sampler.rs:209, -1 if the RNG was not advanced */
    double prob;         /* work[token] / total for a drawn token, else 0 */
    double topp_margin;  /* min_pos |cum - probs[pos] - p| over finite entries (sampler.rs:150), +inf if inactive */
    double cdf_margin;   /* distance of r to the nearest CDF boundary / total (sampler.rs:209-215), +inf if no draw */
    uint64_t kept;       /* entries still finite after top-k / top-p, on the
                            draw and walk-overshoot paths; 0 on the others */
    uint32_t path;       /* ORACLE_PATH_* */
    uint32_t token;
} oracle_stats;

/* Rng::new — sampler.rs:46-56 */
void oracle_rng_new(uint64_t seed, uint64_t state[4]);
/* Rng::next_u64 — sampler.rs:58-72 */
uint64_t oracle_rng_next_u64(uint64_t state[4]);
/* Rng::next_f64 — sampler.rs:75-77 */
double oracle_rng_next_f64(uint64_t state[4]);

/* apply_repetition_penalty — sampler.rs:83-101 */
void oracle_apply_repetition_penalty(double* logits, size_t n, const uint32_t* generated,
                                     size_t n_generated, float penalty);
/* top_k_filter — sampler.rs:103-116 */
void oracle_top_k_filter(double* logits, size_t n, uint64_t k);
/* top_p_filter — sampler.rs:118-160.  `margin_out` (nullable) receives
 * min |cum - probs[pos] - p| over finite entries; `sum_out` the sorted sum. */
void oracle_top_p_filter(double* logits, size_t n, double p, double* margin_out, double* sum_out);

/* sample — sampler.rs:163-217.  `stats` may be NULL. */
uint32_t oracle_sample(const float* logits, size_t n, const oracle_params* params,
                       const uint32_t* generated, size_t n_generated, uint64_t state[4],
                       oracle_stats* stats);

/* Batched driver: row b reads logits + b*ld, advances states[4*b..4*b+3] and
 * penalises generated ids gen_ids[gen_offsets[b] .. gen_offsets[b+1]) (both
 * may be NULL).  Rows are spread over threads exactly like threads.rs
 * par_range(B, 1, ..) (threads.rs:12-61): workers = n_threads if > 0, else
 * NIMBUS_THREADS, else all logical cores; 2*workers chunks; one thread per
 * chunk; inline when B <= 1 or one worker.  Returns the worker count used. */
int oracle_sample_batch(const float* logits, int64_t ld, int32_t B, int64_t V,
                        const oracle_params* params, uint64_t* states,
                        const uint32_t* gen_ids, const int64_t* gen_offsets,
                        uint32_t* tokens, oracle_stats* stats, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
