/* nimbus_sampler.hpp — C++ host mirror of the reference's sampling API
 * (src/sampler.rs) over the C ABI of nimbus_sampler.h.
 *
 * Names, fields, defaults and argument meaning follow the reference:
 *   SamplingParams        src/sampler.rs:7-35   (same fields and Default)
 *   Rng                   src/sampler.rs:41-81  (Rng::new / next_u64 / next_f64)
 *   sample()              src/sampler.rs:163-217 (one host row -> one token id)
 *   apply_repetition_penalty  src/sampler.rs:83-101 (device f64 row)
 * plus Sampler, a device context for the batched entry points.  Every call
 * that reaches the GPU goes through the HIP library; a failed call throws
 * nimbus::Error with the library's status and message (the reference's
 * sample() has no error path; here a device or argument fault surfaces as an
 * exception instead of a wrong token).  Header-only: link
 * libnimbus_sampler.so.
 */
#ifndef NIMBUS_SAMPLER_HPP
#define NIMBUS_SAMPLER_HPP

#include <array>
#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "nimbus_sampler.h"

namespace nimbus {

class Error : public std::runtime_error {
  public:
    Error(int status, const std::string& what) : std::runtime_error(what), status_(status) {}
    int status() const { return status_; }

  private:
    int status_;
};

// src/sampler.rs:7-35.  max_new_tokens, seed and stop_tokens belong to the
// generation loop around sample() and are carried for parity of the type.
struct SamplingParams {
    std::size_t max_new_tokens = 64;
    float temperature = 1.0f;
    std::size_t top_k = 0;       // 0 disables
    float top_p = 1.0f;          // 1.0 disables
    float repetition_penalty = 1.0f;
    std::optional<uint64_t> seed;
    std::vector<uint32_t> stop_tokens;

    bool greedy() const { return temperature <= 0.0f; }

    nis_params to_c() const {
        nis_params p{};
        p.temperature = temperature;
        p.top_p = top_p;
        p.repetition_penalty = repetition_penalty;
        p.reserved = 0;
        p.top_k = static_cast<uint64_t>(top_k);
        return p;
    }
};

// src/sampler.rs:41-81: xoshiro256++ seeded through SplitMix64.
class Rng {
  public:
    explicit Rng(uint64_t seed) { nis_rng_seed(seed, state_.data()); }
    static Rng from_state(const std::array<uint64_t, 4>& s) {
        Rng r(0);
        r.state_ = s;
        return r;
    }
    uint64_t next_u64() { return nis_rng_next_u64(state_.data()); }
    double next_f64() { return nis_rng_next_f64(state_.data()); }
    const std::array<uint64_t, 4>& state() const { return state_; }
    std::array<uint64_t, 4>& state() { return state_; }

  private:
    std::array<uint64_t, 4> state_{};
};

// A device context (own default-priority stream unless set_stream is used).
class Sampler {
  public:
    explicit Sampler(int device = 0) { check(nis_ctx_create(device, &ctx_), "nis_ctx_create"); }
    ~Sampler() {
        if (ctx_) (void)nis_ctx_destroy(ctx_);
    }
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;
    Sampler(Sampler&& o) noexcept : ctx_(o.ctx_) { o.ctx_ = nullptr; }

    nis_ctx* handle() const { return ctx_; }
    void set_stream(void* hip_stream) { check(nis_ctx_set_stream(ctx_, hip_stream), "set_stream"); }
    void* stream() const { return nis_ctx_get_stream(ctx_); }
    void sync() { check(nis_sync(ctx_), "sync"); }

    // sample() of src/sampler.rs:163 on one host row; advances `rng` exactly
    // as the reference does (once, iff the row reaches the draw).
    uint32_t sample(const float* logits, std::size_t V, const SamplingParams& params,
                    const uint32_t* generated, std::size_t n_generated, Rng& rng) {
        const nis_params p = params.to_c();
        uint32_t tok = 0;
        check(nis_sample_one(ctx_, logits, static_cast<int64_t>(V), &p, generated,
                             static_cast<int64_t>(n_generated), rng.state().data(), &tok),
              "sample");
        return tok;
    }
    uint32_t sample(const std::vector<float>& logits, const SamplingParams& params,
                    const std::vector<uint32_t>& generated, Rng& rng) {
        return sample(logits.data(), logits.size(), params, generated.data(), generated.size(), rng);
    }

    // Batched sample() over device buffers (asynchronous on stream()).
    void sample_batch(const float* d_logits, int64_t ld, int32_t B, int64_t V,
                      const SamplingParams& params, uint64_t* d_rng_state,
                      const uint32_t* d_gen_ids, const int64_t* d_gen_offsets, uint32_t* d_tokens,
                      nis_row_stats* d_stats = nullptr) {
        const nis_params p = params.to_c();
        check(nis_sample_batch(ctx_, d_logits, ld, B, V, &p, d_rng_state, d_gen_ids, d_gen_offsets,
                               d_tokens, d_stats),
              "sample_batch");
    }
    // Logits of B last-hidden rows (Model::logits_last, model.rs:317-325): see
    // nis_lm_head_logits.  Asynchronous on the context stream.
    void lm_head_logits(const float* d_hidden, int64_t ldh, int32_t B, int32_t H,
                        const nis_weights& w, int64_t V, float* d_logits, int64_t ld) {
        check(nis_lm_head_logits(ctx_, d_hidden, ldh, B, H, &w, V, d_logits, ld), "lm_head_logits");
    }

    // One step of a batched decode loop (engine.rs:279-287): see nis_decode_step.
    void decode_step(const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     const SamplingParams& params, uint64_t* d_rng_state, uint32_t* d_gen_ids,
                     int64_t gen_cap, int32_t* d_gen_len, const int32_t* d_max_new,
                     const uint32_t* d_stop_ids, int32_t n_stop, uint8_t* d_done,
                     uint32_t* d_tokens, nis_row_stats* d_stats = nullptr) {
        const nis_params p = params.to_c();
        check(nis_decode_step(ctx_, d_logits, ld, B, V, &p, d_rng_state, d_gen_ids, gen_cap,
                              d_gen_len, d_max_new, d_stop_ids, n_stop, d_done, d_tokens, d_stats),
              "decode_step");
    }
    void argmax_batch(const float* d_logits, int64_t ld, int32_t B, int64_t V, uint32_t* d_tokens) {
        check(nis_argmax_batch(ctx_, d_logits, ld, B, V, d_tokens), "argmax_batch");
    }
    void rng_seed_batch(const uint64_t* d_seeds, int32_t B, uint64_t* d_states) {
        check(nis_rng_seed_batch(ctx_, d_seeds, B, d_states), "rng_seed_batch");
    }
    // src/sampler.rs:83-101 on a device f64 row.
    void apply_repetition_penalty(double* d_logits, int64_t V, const uint32_t* d_generated,
                                  int64_t n_generated, float penalty) {
        check(nis_apply_repetition_penalty(ctx_, d_logits, V, d_generated, n_generated, penalty),
              "apply_repetition_penalty");
    }

  private:
    void check(int status, const char* what) const {
        if (status == NIS_OK) return;
        std::string msg = std::string(what) + ": " + nis_status_string(status);
        if (ctx_) {
            const char* e = nis_last_error(ctx_);
            if (e && *e) msg += std::string(" (") + e + ")";
        }
        throw Error(status, msg);
    }
    nis_ctx* ctx_ = nullptr;
};

// The reference's free function: sample(logits, params, generated, rng).
// Uses one context per thread on device 0.
inline uint32_t sample(const std::vector<float>& logits, const SamplingParams& params,
                       const std::vector<uint32_t>& generated, Rng& rng) {
    thread_local Sampler s(0);
    return s.sample(logits, params, generated, rng);
}

}  // namespace nimbus

#endif  // NIMBUS_SAMPLER_HPP
