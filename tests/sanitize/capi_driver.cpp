// Drives the host side of the C ABI (include/nimbus_sampler.h,
// nimbus-infer-rs_amd/csrc/capi.hip) under AddressSanitizer and
// UndefinedBehaviorSanitizer (host code only; the device code is built
// without them): the host RNG against the oracle's, status strings, and
// every argument check reachable without a GPU (null contexts and
// pointers, no device).  Exits non-zero on a wrong answer; a sanitizer
// report aborts (built with -fno-sanitize-recover=all).
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "nimbus_sampler.h"

extern "C" {
void oracle_rng_new(uint64_t seed, uint64_t state[4]);
uint64_t oracle_rng_next_u64(uint64_t state[4]);
double oracle_rng_next_f64(uint64_t state[4]);
}

#define CHECK(c)                                                             \
    do {                                                                     \
        if (!(c)) {                                                          \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            return 1;                                                        \
        }                                                                    \
    } while (0)

int main() {
    // Rng::new / next_u64 / next_f64 against the oracle
    uint64_t seed = 0x5DEECE66Dull;
    for (int i = 0; i < 2000; ++i) {
        uint64_t a[4], b[4];
        nis_rng_seed(seed, a);
        oracle_rng_new(seed, b);
        CHECK(std::memcmp(a, b, sizeof(a)) == 0);
        for (int j = 0; j < 8; ++j) CHECK(nis_rng_next_u64(a) == oracle_rng_next_u64(b));
        CHECK(nis_rng_next_f64(a) == oracle_rng_next_f64(b));
        seed = seed * 6364136223846793005ull + 1442695040888963407ull;
    }
    nis_rng_seed(1, nullptr);
    CHECK(nis_rng_next_u64(nullptr) == 0);
    for (int s = -6; s <= 2; ++s) CHECK(nis_status_string(s) != nullptr);
    // no context / no device
    CHECK(nis_ctx_create(0, nullptr) == NIS_EINVAL);
    nis_ctx* ctx = nullptr;
    const int rc = nis_ctx_create(-1, &ctx);
    CHECK(rc == NIS_ENODEV && ctx == nullptr);
    CHECK(nis_ctx_destroy(nullptr) == NIS_EINVAL);
    CHECK(std::strcmp(nis_last_error(nullptr), "") == 0);
    CHECK(nis_ctx_get_stream(nullptr) == nullptr);
    nis_params p{};
    p.temperature = 0.8f;
    p.top_p = 0.9f;
    p.repetition_penalty = 1.0f;
    float logits[8] = {0, 1, 2, 3, 4, 5, 6, 7};
    uint64_t st[4];
    uint32_t tok = 0;
    nis_rng_seed(7, st);
    CHECK(nis_sample_batch(nullptr, logits, 8, 1, 8, &p, st, nullptr, nullptr, &tok, nullptr) == NIS_EINVAL);
    CHECK(nis_sample_one(nullptr, logits, 8, &p, nullptr, 0, st, &tok) == NIS_EINVAL);
    CHECK(nis_sample_one_noalloc(nullptr, logits, 8, &p, nullptr, 0, st, &tok) == NIS_EINVAL);
    CHECK(nis_argmax_batch(nullptr, logits, 8, 1, 8, &tok) == NIS_EINVAL);
    CHECK(nis_sync(nullptr) == NIS_EINVAL);
    CHECK(nis_rng_seed_batch(nullptr, st, 1, st) == NIS_EINVAL);
    std::printf("C ABI sanitizer driver: clean\n");
    return 0;
}
