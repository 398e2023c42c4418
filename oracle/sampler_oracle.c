/*
 * sampler_oracle.c — CPU restatement of nimbus-infer-rs `src/sampler.rs`
 * (plus the fork-join of `src/threads.rs` for the batched CPU baseline).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP sampler and the timed
 * CPU baseline.  Never linked into, called by, or used as a fallback of the
 * product library.
 *
 * Build: gcc -O2 -std=c11 -fno-fast-math -ffp-contract=off -fPIC -shared
 *        (oracle/build_oracle.py).  f64 throughout, glibc `exp` (the libm
 * routine Rust's f64::exp lowers to on Linux x86-64), sequential sums in the
 * reference's order, a stable merge sort where the reference uses `sort_by`.
 *
 * Pinning (what checks this restatement, see tests/test_oracle.py):
 *   - Rng::new / next_u64 / next_f64: the published SplitMix64(0) stream
 *     (state = outputs #2..#5), an independent Python big-int restatement's
 *     known-answer vectors (tests/golden/rng_kats.json), the GF(2)-linearity
 *     of the xoshiro state transition, and the reference test
 *     `rng_is_deterministic_and_seeded` (sampler.rs:230-239).
 *   - greedy: reference test `greedy_takes_first_max` (sampler.rs:223-228)
 *     and brute-force first-index argmax.
 *   - top_k_filter: reference test `top_k_keeps_only_best_k`
 *     (sampler.rs:241-249) and brute force over tiny rows.
 *   - top_p_filter: reference test `top_p_zero_keeps_argmax_only`
 *     (sampler.rs:259-266); for 0<p<1 an exact-rational (Fraction) evaluation
 *     of the rule at sampler.rs:147-154 on tiny rows away from boundaries.
 *   - apply_repetition_penalty: reference test
 *     `repetition_penalty_divides_positive_multiplies_negative` (251-257).
 *   - temperature/softmax/draw: closed-form inverse CDF on tiny rows with
 *     u placed just inside / outside each cumulative boundary.
 *   The bit-level f64 rounding of the sequential cumsum and walk, and the
 *   value of libm `exp`, are pinned only by restatement (no reference
 *   golden holds them); the GPU is compared to them with the stated
 *   1e-6 boundary tolerance.
 */
#define _GNU_SOURCE
#include "sampler_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* RNG: SplitMix64-seeded xoshiro256++ (Steele/Lea/Flood 2014; Blackman and
 * Vigna 2018).  The reference pre-increments its SplitMix counter once
 * before the first draw (sampler.rs:47 then 49), so the state is SplitMix64
 * outputs #2..#5. */

#define GOLDEN_GAMMA 0x9E3779B97F4A7C15ULL

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void oracle_rng_new(uint64_t seed, uint64_t state[4]) {
    uint64_t sm = seed + GOLDEN_GAMMA;                 /* sampler.rs:47 */
    for (int i = 0; i < 4; ++i) {                      /* sampler.rs:48-55 */
        sm += GOLDEN_GAMMA;
        uint64_t z = sm;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        state[i] = z ^ (z >> 31);
    }
}

uint64_t oracle_rng_next_u64(uint64_t s[4]) {
    const uint64_t result = rotl64(s[0] + s[3], 23) + s[0];   /* sampler.rs:59-63 */
    const uint64_t t = s[1] << 17;                             /* 64 */
    s[2] ^= s[0];                                              /* 65 */
    s[3] ^= s[1];                                              /* 66 */
    s[1] ^= s[2];                                              /* 67 */
    s[0] ^= s[3];                                              /* 68 */
    s[2] ^= t;                                                 /* 69 */
    s[3] = rotl64(s[3], 45);                                   /* 70 */
    return result;
}

double oracle_rng_next_f64(uint64_t s[4]) {
    /* sampler.rs:76: (x >> 11) as f64 * (1.0 / 2^53) — exact */
    return (double)(oracle_rng_next_u64(s) >> 11) * (1.0 / 9007199254740992.0);
}

/* ------------------------------------------------------------------------ */
/* Filters */

static int cmp_u32(const void* a, const void* b) {
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return (x > y) - (x < y);
}

void oracle_apply_repetition_penalty(double* logits, size_t n, const uint32_t* generated,
                                     size_t n_generated, float penalty) {
    if (penalty == 1.0f || n_generated == 0) return;            /* sampler.rs:84-86 */
    uint32_t* seen = (uint32_t*)malloc(n_generated * sizeof(uint32_t));
    memcpy(seen, generated, n_generated * sizeof(uint32_t));
    qsort(seen, n_generated, sizeof(uint32_t), cmp_u32);        /* 87-88 */
    size_t m = 0;                                               /* 89: dedup */
    for (size_t i = 0; i < n_generated; ++i)
        if (m == 0 || seen[m - 1] != seen[i]) seen[m++] = seen[i];
    const double pen = (double)penalty;
    for (size_t i = 0; i < m; ++i) {                            /* 90-100 */
        size_t idx = seen[i];
        if (idx >= n) continue;
        if (logits[idx] > 0.0) logits[idx] /= pen;
        else logits[idx] *= pen;
    }
    free(seen);
}

/* partial_cmp(a, b).unwrap_or(Equal) as -1/0/+1 */
static int partial_cmp(double a, double b) {
    if (a < b) return -1;
    if (a > b) return 1;
    return 0;
}

static int cmp_desc_f64(const void* pa, const void* pb) {
    /* sampler.rs:109: |a, b| b.partial_cmp(a) */
    return partial_cmp(*(const double*)pb, *(const double*)pa);
}

void oracle_top_k_filter(double* logits, size_t n, uint64_t k) {
    if (k == 0 || k >= n) return;                               /* sampler.rs:104-106 */
    double* sorted = (double*)malloc(n * sizeof(double));       /* 108 */
    memcpy(sorted, logits, n * sizeof(double));
    qsort(sorted, n, sizeof(double), cmp_desc_f64);             /* 109 */
    const double kth = sorted[k - 1];                           /* 110 */
    for (size_t i = 0; i < n; ++i)                              /* 111-115 */
        if (logits[i] < kth) logits[i] = -INFINITY;
    free(sorted);
}

/* Stable descending merge sort of indices by logits[i] (sampler.rs:140,
 * `sort_by` is stable: equal keys keep ascending index order). */
static void merge_sort_idx(size_t* a, size_t* tmp, size_t n, const double* key) {
    for (size_t width = 1; width < n; width *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * width) {
            size_t mid = lo + width < n ? lo + width : n;
            size_t hi = lo + 2 * width < n ? lo + 2 * width : n;
            size_t i = lo, j = mid, o = lo;
            while (i < mid && j < hi) {
                /* take from the right run only if it is strictly "less" in the
                 * descending order, i.e. key[right] > key[left] */
                if (partial_cmp(key[a[i]], key[a[j]]) < 0) tmp[o++] = a[j++];
                else tmp[o++] = a[i++];
            }
            while (i < mid) tmp[o++] = a[i++];
            while (j < hi) tmp[o++] = a[j++];
        }
        memcpy(a, tmp, n * sizeof(size_t));
    }
}

void oracle_top_p_filter(double* logits, size_t n, double p, double* margin_out, double* sum_out) {
    if (margin_out) *margin_out = INFINITY;
    if (sum_out) *sum_out = 0.0;
    if (p >= 1.0) return;                                       /* sampler.rs:119-121 */
    if (p <= 0.0) {                                             /* 122-135 */
        /* Iterator::max_by keeps the LAST of equal maxima: it replaces the
         * running best unless best compares Greater than the candidate. */
        size_t best = 0;
        for (size_t i = 1; i < n; ++i)
            if (!(partial_cmp(logits[best], logits[i]) > 0)) best = i;
        if (n == 0) return;
        const double keep = logits[best];
        for (size_t i = 0; i < n; ++i) logits[i] = -INFINITY;
        logits[best] = keep;
        return;
    }
    if (n == 0) return; /* the reference panics at order[0] (sampler.rs:141) */
    size_t* order = (size_t*)malloc(n * sizeof(size_t));        /* 139 */
    size_t* tmp = (size_t*)malloc(n * sizeof(size_t));
    for (size_t i = 0; i < n; ++i) order[i] = i;
    merge_sort_idx(order, tmp, n, logits);                      /* 140 */
    const double max = logits[order[0]];                        /* 141 */
    double* probs = (double*)malloc(n * sizeof(double));
    for (size_t pos = 0; pos < n; ++pos)                        /* 142 */
        probs[pos] = exp(logits[order[pos]] - max);
    double sum = 0.0;                                           /* 143: sequential */
    for (size_t pos = 0; pos < n; ++pos) sum += probs[pos];
    for (size_t pos = 0; pos < n; ++pos) probs[pos] /= sum;     /* 144-146 */
    double cum = 0.0;                                           /* 147 */
    unsigned char* remove = (unsigned char*)calloc(n, 1);       /* 148 */
    double margin = INFINITY;
    for (size_t pos = 0; pos < n; ++pos) {                      /* 149-154 */
        const size_t i = order[pos];
        const double d = cum - probs[pos];
        if (d > p) remove[i] = 1;
        if (isfinite(logits[i])) {
            double m = fabs(d - p);
            if (m < margin) margin = m;
        }
        cum += probs[pos];
    }
    for (size_t i = 0; i < n; ++i)                              /* 155-159 */
        if (remove[i]) logits[i] = -INFINITY;
    if (margin_out) *margin_out = margin;
    if (sum_out) *sum_out = sum;
    free(remove);
    free(probs);
    free(tmp);
    free(order);
}

/* ------------------------------------------------------------------------ */
/* sample — sampler.rs:163-217 */

static size_t first_argmax(const double* w, size_t n) {
    size_t best = 0;                      /* sampler.rs:174-179 / 193-198 */
    for (size_t i = 0; i < n; ++i)
        if (w[i] > w[best]) best = i;
    return best;
}

uint32_t oracle_sample(const float* logits, size_t n, const oracle_params* params,
                       const uint32_t* generated, size_t n_generated, uint64_t state[4],
                       oracle_stats* stats) {
    oracle_stats st;
    memset(&st, 0, sizeof st);
    st.u = -1.0;
    st.topp_margin = INFINITY;
    st.cdf_margin = INFINITY;

    double* work = (double*)malloc((n ? n : 1) * sizeof(double));
    for (size_t i = 0; i < n; ++i) work[i] = (double)logits[i];            /* 169 */
    oracle_apply_repetition_penalty(work, n, generated, n_generated,
                                    params->repetition_penalty);          /* 170 */
    uint32_t token;

    if (params->temperature <= 0.0f) {                                      /* 32-34, 172 */
        token = (uint32_t)first_argmax(work, n);
        st.path = ORACLE_PATH_GREEDY;
        goto done;
    }
    {
        /* f64::max(T, 1e-6): returns the non-NaN operand, like C fmax */
        const double temp = fmax((double)params->temperature, 1e-6);      /* 183 */
        for (size_t i = 0; i < n; ++i) work[i] /= temp;                    /* 184-186 */
        oracle_top_k_filter(work, n, params->top_k);                        /* 187 */
        oracle_top_p_filter(work, n, (double)params->top_p, &st.topp_margin,
                            &st.z_sorted);                                  /* 188 */

        double max = -INFINITY;                                            /* 191 */
        for (size_t i = 0; i < n; ++i) max = fmax(max, work[i]);
        st.max_w = max;
        if (!isfinite(max)) {                                              /* 192-200 */
            token = (uint32_t)first_argmax(work, n);
            st.path = ORACLE_PATH_NONFINITE_MAX;
            goto done;
        }
        uint64_t kept = 0;  /* entries still finite after the filters */
        for (size_t i = 0; i < n; ++i) kept += isfinite(work[i]) ? 1 : 0;
        double total = 0.0;                                                /* 201-205 */
        for (size_t i = 0; i < n; ++i) {
            work[i] = exp(work[i] - max);
            total += work[i];
        }
        st.z_kept = total;
        if (!isfinite(total) || total <= 0.0) {                            /* 206-208 */
            token = 0;
            st.path = ORACLE_PATH_BAD_TOTAL;
            goto done;
        }
        st.kept = kept;  /* reported on the draw paths only (0 on the ones above) */
        const double u = oracle_rng_next_f64(state);                      /* 209 */
        double r = u * total;
        st.u = u;
        for (size_t i = 0; i < n; ++i) {                                   /* 210-215 */
            const double before = r;
            r -= work[i];
            if (r <= 0.0) {
                token = (uint32_t)i;
                st.path = ORACLE_PATH_DRAW;
                st.prob = work[i] / total;
                st.cdf_margin = fmin(before, -r) / total;
                goto done;
            }
        }
        token = (uint32_t)(n - 1);                                          /* 216 */
        st.path = ORACLE_PATH_FALLTHROUGH;
        st.prob = work[n - 1] / total;
        st.cdf_margin = r / total;
    }
done:
    free(work);
    st.token = token;
    if (stats) *stats = st;
    return token;
}

/* ------------------------------------------------------------------------ */
/* Batched CPU baseline over threads.rs-style fork-join */

typedef struct batch_job {
    const float* logits;
    int64_t ld;
    int64_t V;
    const oracle_params* params;
    uint64_t* states;
    const uint32_t* gen_ids;
    const int64_t* gen_offsets;
    uint32_t* tokens;
    oracle_stats* stats;
    int64_t start, end;
} batch_job;

static void run_rows(const batch_job* j) {
    for (int64_t b = j->start; b < j->end; ++b) {
        const uint32_t* g = NULL;
        size_t ng = 0;
        if (j->gen_ids && j->gen_offsets) {
            g = j->gen_ids + j->gen_offsets[b];
            ng = (size_t)(j->gen_offsets[b + 1] - j->gen_offsets[b]);
        }
        j->tokens[b] = oracle_sample(j->logits + b * j->ld, (size_t)j->V, j->params, g, ng,
                                     j->states + 4 * b, j->stats ? j->stats + b : NULL);
    }
}

static void* run_rows_thread(void* arg) {
    run_rows((const batch_job*)arg);
    return NULL;
}

/* threads.rs:12-26 */
static int worker_count(void) {
    const char* env = getenv("NIMBUS_THREADS");
    if (env) {
        char* end = NULL;
        long v = strtol(env, &end, 10);
        if (end && *end == '\0' && end != env && v > 0) return (int)v;
    }
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

int oracle_sample_batch(const float* logits, int64_t ld, int32_t B, int64_t V,
                        const oracle_params* params, uint64_t* states,
                        const uint32_t* gen_ids, const int64_t* gen_offsets,
                        uint32_t* tokens, oracle_stats* stats, int n_threads) {
    batch_job base = {logits, ld, V, params, states, gen_ids, gen_offsets, tokens, stats, 0, B};
    const int64_t n = B, min_chunk = 1;
    const int workers = n_threads > 0 ? n_threads : worker_count();
    if (n <= min_chunk || workers <= 1) {               /* threads.rs:34-37 */
        run_rows(&base);
        return 1;
    }
    const int64_t target_chunks = (int64_t)workers * 2; /* 38-39 */
    int64_t chunk = (n + target_chunks - 1) / target_chunks;
    if (chunk < min_chunk) chunk = min_chunk;
    const int64_t n_chunks = (n + chunk - 1) / chunk;
    pthread_t* th = (pthread_t*)malloc((size_t)n_chunks * sizeof(pthread_t));
    batch_job* jobs = (batch_job*)malloc((size_t)n_chunks * sizeof(batch_job));
    int64_t c = 0;
    for (int64_t start = 0; start < n; start += chunk, ++c) {   /* 41-48 */
        jobs[c] = base;
        jobs[c].start = start;
        jobs[c].end = start + chunk < n ? start + chunk : n;
        pthread_create(&th[c], NULL, run_rows_thread, &jobs[c]);
    }
    for (int64_t i = 0; i < c; ++i) pthread_join(th[i], NULL); /* 49-51 */
    free(jobs);
    free(th);
    return workers;
}
