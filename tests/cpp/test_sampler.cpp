// C++ mirror of the reference's unit tests (src/sampler.rs:223-266) through
// the C++ host API (include/nimbus_sampler.hpp) and the HIP library.
//
//   test_sampler cpu   host-only checks (Rng, SamplingParams)
//   test_sampler gpu   checks that run the HIP sampler on device 0
//
// Exit status 0 when every check passes; each failure prints its line.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <set>
#include <vector>

#include "nimbus_sampler.hpp"

static int g_failures = 0;
#define CHECK(cond)                                                          \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);      \
            ++g_failures;                                                    \
        }                                                                    \
    } while (0)

// sampler.rs:231 rng_is_deterministic_and_seeded
static void rng_is_deterministic_and_seeded() {
    nimbus::Rng a(42), b(42);
    for (int i = 0; i < 100; ++i) CHECK(a.next_u64() == b.next_u64());
    nimbus::Rng c(43);
    CHECK(a.next_u64() != c.next_u64());
}

// SamplingParams::default and greedy() (sampler.rs:17-35)
static void params_defaults() {
    nimbus::SamplingParams p;
    CHECK(p.max_new_tokens == 64);
    CHECK(p.temperature == 1.0f);
    CHECK(p.top_k == 0);
    CHECK(p.top_p == 1.0f);
    CHECK(p.repetition_penalty == 1.0f);
    CHECK(!p.seed.has_value());
    CHECK(p.stop_tokens.empty());
    CHECK(!p.greedy());
    p.temperature = 0.0f;
    CHECK(p.greedy());
    p.temperature = -1.0f;
    CHECK(p.greedy());
}

// next_f64 is the top 53 bits of next_u64 scaled by 2^-53 (sampler.rs:75-77)
static void next_f64_is_top_53_bits() {
    nimbus::Rng a(7), b(7);
    for (int i = 0; i < 64; ++i) {
        const uint64_t u = a.next_u64();
        const double f = b.next_f64();
        CHECK(f == (double)(u >> 11) * 0x1.0p-53);
        CHECK(f >= 0.0 && f < 1.0);
    }
}

// sampler.rs:224 greedy_takes_first_max
static void greedy_takes_first_max(nimbus::Sampler& s) {
    nimbus::SamplingParams p;
    p.temperature = 0.0f;
    nimbus::Rng rng(0);
    const auto before = rng.state();
    CHECK(s.sample({0.1f, 5.0f, 5.0f, -1.0f}, p, {}, rng) == 1);
    CHECK(rng.state() == before);  // greedy never draws
}

// sampler.rs:242 top_k_keeps_only_best_k: with k = 2 only ids 1 (5.0) and
// 3 (4.0) survive the filter, so no seed can draw 0 or 2, and both occur
static void top_k_keeps_only_best_k(nimbus::Sampler& s) {
    nimbus::SamplingParams p;
    p.temperature = 1.0f;
    p.top_k = 2;
    std::set<uint32_t> seen;
    for (uint64_t seed = 0; seed < 64; ++seed) {
        nimbus::Rng rng(seed);
        seen.insert(s.sample({1.0f, 5.0f, 3.0f, 4.0f}, p, {}, rng));
    }
    CHECK(seen == (std::set<uint32_t>{1, 3}));
}

// sampler.rs:252 repetition_penalty_divides_positive_multiplies_negative
static void repetition_penalty(nimbus::Sampler& s) {
    const double h[2] = {2.0, -2.0};
    const uint32_t g[2] = {0, 1};
    double* d = nullptr;
    uint32_t* dg = nullptr;
    CHECK(hipMalloc(&d, sizeof h) == hipSuccess);
    CHECK(hipMalloc(&dg, sizeof g) == hipSuccess);
    CHECK(hipMemcpy(d, h, sizeof h, hipMemcpyHostToDevice) == hipSuccess);
    CHECK(hipMemcpy(dg, g, sizeof g, hipMemcpyHostToDevice) == hipSuccess);
    s.apply_repetition_penalty(d, 2, dg, 2, 2.0f);
    s.sync();
    double out[2] = {0, 0};
    CHECK(hipMemcpy(out, d, sizeof out, hipMemcpyDeviceToHost) == hipSuccess);
    CHECK(out[0] == 1.0);
    CHECK(out[1] == -4.0);
    (void)hipFree(d);
    (void)hipFree(dg);
}

// sampler.rs:260 top_p_zero_keeps_argmax_only: only id 1 survives
static void top_p_zero_keeps_argmax_only(nimbus::Sampler& s) {
    nimbus::SamplingParams p;
    p.temperature = 1.0f;
    p.top_p = 0.0f;
    for (uint64_t seed = 0; seed < 32; ++seed) {
        nimbus::Rng rng(seed);
        CHECK(s.sample({1.0f, 5.0f, 3.0f}, p, {}, rng) == 1);
    }
}

// same seed, same token and the same single RNG advance
static void sample_is_deterministic(nimbus::Sampler& s) {
    std::vector<float> x(50257);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.37f * (float)i) * 3.0f;
    nimbus::SamplingParams p;
    p.temperature = 0.8f;
    p.top_p = 0.9f;
    nimbus::Rng a(11), b(11), expect(11);
    const uint32_t ta = s.sample(x, p, {}, a);
    const uint32_t tb = nimbus::sample(x, p, {}, b);  // the free function
    CHECK(ta == tb);
    CHECK(ta < x.size());
    expect.next_u64();
    CHECK(a.state() == expect.state());
    CHECK(b.state() == expect.state());
}

// simd.rs:183 dot_f32_matches_scalar and simd.rs:192 dot_i8_matches_reference,
// through the LM-head producer (one weight row, one hidden row)
static float lm_head_one(nimbus::Sampler& s, const std::vector<float>& x, const void* w,
                         size_t wbytes, int32_t format) {
    const int32_t H = (int32_t)x.size();
    float *dx = nullptr, *ds = nullptr, *dout = nullptr;
    void* dw = nullptr;
    const float one = 1.0f;
    CHECK(hipMalloc(&dx, x.size() * sizeof(float)) == hipSuccess);
    CHECK(hipMalloc(&dw, wbytes) == hipSuccess);
    CHECK(hipMalloc(&ds, sizeof one) == hipSuccess);
    CHECK(hipMalloc(&dout, sizeof(float)) == hipSuccess);
    CHECK(hipMemcpy(dx, x.data(), x.size() * sizeof(float), hipMemcpyHostToDevice) == hipSuccess);
    CHECK(hipMemcpy(dw, w, wbytes, hipMemcpyHostToDevice) == hipSuccess);
    CHECK(hipMemcpy(ds, &one, sizeof one, hipMemcpyHostToDevice) == hipSuccess);
    nis_weights wt;
    wt.format = format;
    wt.group_size = 0;
    wt.d_data = dw;
    wt.d_scales = format == NIS_W_F32 ? nullptr : ds;
    s.lm_head_logits(dx, H, 1, H, wt, 1, dout, 1);
    s.sync();
    float out = 0.0f;
    CHECK(hipMemcpy(&out, dout, sizeof out, hipMemcpyDeviceToHost) == hipSuccess);
    (void)hipFree(dx);
    (void)hipFree(dw);
    (void)hipFree(ds);
    (void)hipFree(dout);
    return out;
}

static void lm_head_matches_reference_dots(nimbus::Sampler& s) {
    std::vector<float> a(257), b(257);
    double exact = 0.0;
    for (int i = 0; i < 257; ++i) {
        a[i] = (float)i * 0.5f - 30.0f;
        b[i] = 1.0f / ((float)i + 3.0f);
        exact += (double)a[i] * (double)b[i];
    }
    CHECK(std::fabs(lm_head_one(s, a, b.data(), b.size() * sizeof(float), NIS_W_F32) - exact) < 1e-2);
    std::vector<float> x(131);
    std::vector<uint8_t> q(131);
    exact = 0.0;
    for (int i = 0; i < 131; ++i) {
        x[i] = (float)i * 0.125f;
        const int raw = (i * 7) % 255 - 128;
        q[i] = (uint8_t)(raw + 128);
        exact += (double)x[i] * raw;
    }
    CHECK(std::fabs(lm_head_one(s, x, q.data(), q.size(), NIS_W_INT8) - exact) < 1e-2);
}

static void errors_throw(nimbus::Sampler& s) {
    nimbus::SamplingParams p;
    nimbus::Rng rng(0);
    bool threw = false;
    try {
        s.sample(nullptr, 0, p, nullptr, 0, rng);  // V = 0 is invalid
    } catch (const nimbus::Error& e) {
        threw = e.status() != NIS_OK;
    }
    CHECK(threw);
}

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
    rng_is_deterministic_and_seeded();
    params_defaults();
    next_f64_is_top_53_bits();
    if (gpu) {
        nimbus::Sampler s(0);
        greedy_takes_first_max(s);
        top_k_keeps_only_best_k(s);
        repetition_penalty(s);
        top_p_zero_keeps_argmax_only(s);
        sample_is_deterministic(s);
        lm_head_matches_reference_dots(s);
        errors_throw(s);
    }
    std::printf("%s: %d failure(s)\n", gpu ? "gpu" : "cpu", g_failures);
    return g_failures == 0 ? 0 : 1;
}
