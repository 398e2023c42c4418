/* Drives the CPU oracle (oracle/sampler_oracle.c) under AddressSanitizer and
 * UndefinedBehaviorSanitizer: random rows of many shapes and the special
 * rows of sampler.rs (NaN, +-inf, all -inf, ties, u = 0 territory) through
 * every branch of sample() and the threads.rs batch driver.  Exits non-zero
 * on any sanitizer report (built with -fno-sanitize-recover=all). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sampler_oracle.h"

static uint64_t g_s = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) {
    g_s ^= g_s << 13;
    g_s ^= g_s >> 7;
    g_s ^= g_s << 17;
    return g_s;
}
static float unif(void) { return (float)((rnd() >> 11) * (1.0 / 9007199254740992.0)); }

int main(void) {
    const size_t sizes[] = {1, 2, 3, 7, 64, 257, 4099};
    const float temps[] = {0.0f, 1e-7f, 0.3f, 1.0f, 1.7f};
    const float tops[] = {0.0f, 0.37f, 0.9f, 0.999f, 1.0f};
    const uint64_t ks[] = {0, 1, 3, 50, 1u << 20};
    const float pens[] = {1.0f, 0.8f, 1.3f};
    unsigned long long checked = 0;
    for (size_t si = 0; si < sizeof(sizes) / sizeof(sizes[0]); ++si) {
        const size_t V = sizes[si];
        float* x = (float*)malloc(V * sizeof(float));
        uint32_t* gen = (uint32_t*)malloc(8 * sizeof(uint32_t));
        for (int rep = 0; rep < 24; ++rep) {
            for (size_t i = 0; i < V; ++i) x[i] = (unif() - 0.5f) * 12.0f;
            switch (rep % 8) {
                case 1: x[rnd() % V] = NAN; break;
                case 2: x[rnd() % V] = INFINITY; break;
                case 3: for (size_t i = 0; i < V; ++i) x[i] = -INFINITY; break;
                case 4: for (size_t i = 0; i < V; ++i) x[i] = (float)(int)(x[i] / 3.0f); break;
                case 5: x[rnd() % V] = -INFINITY; break;
                default: break;
            }
            for (int g = 0; g < 8; ++g) gen[g] = (uint32_t)(rnd() % (V + 2));
            for (size_t ti = 0; ti < 5; ++ti)
                for (size_t pi = 0; pi < 5; ++pi)
                    for (size_t ki = 0; ki < 5; ++ki)
                        for (size_t ni = 0; ni < 3; ++ni) {
                            oracle_params p;
                            memset(&p, 0, sizeof(p));
                            p.temperature = temps[ti];
                            p.top_p = tops[pi];
                            p.top_k = ks[ki];
                            p.repetition_penalty = pens[ni];
                            uint64_t st[4];
                            oracle_rng_new(rnd(), st);
                            oracle_stats s;
                            const uint32_t tok = oracle_sample(x, V, &p, gen, (size_t)(rep % 9), st, &s);
                            if (tok >= V) {
                                fprintf(stderr, "token %u out of range for V=%zu\n", tok, V);
                                return 2;
                            }
                            ++checked;
                        }
        }
        /* the batch driver over 16 rows with CSR histories, several threads */
        const int B = 16;
        float* xb = (float*)malloc((size_t)B * V * sizeof(float));
        for (size_t i = 0; i < (size_t)B * V; ++i) xb[i] = (unif() - 0.5f) * 8.0f;
        uint64_t* states = (uint64_t*)malloc(4 * (size_t)B * sizeof(uint64_t));
        int64_t off[17];
        uint32_t ids[16 * 3];
        off[0] = 0;
        for (int b = 0; b < B; ++b) {
            off[b + 1] = off[b] + (b % 4);
            for (int64_t j = off[b]; j < off[b + 1]; ++j) ids[j] = (uint32_t)(rnd() % V);
            oracle_rng_new((uint64_t)b, states + 4 * b);
        }
        uint32_t tokens[16];
        oracle_stats stats[16];
        oracle_params p;
        memset(&p, 0, sizeof(p));
        p.temperature = 0.8f;
        p.top_p = 0.9f;
        p.repetition_penalty = 1.3f;
        oracle_sample_batch(xb, (int64_t)V, B, (int64_t)V, &p, states, ids, off, tokens, stats, 4);
        for (int b = 0; b < B; ++b)
            if (tokens[b] >= V) return 3;
        free(xb);
        free(states);
        free(x);
        free(gen);
    }
    printf("oracle sanitizer driver: %llu sample() calls clean\n", checked);
    return 0;
}
