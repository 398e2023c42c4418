/*
 * nimbus_sampler.h — C ABI of the MI355X (gfx950) token sampler.
 *
 * Drop-in boundary for nimbus-infer-rs `src/sampler.rs`: every entry point
 * below replaces one item of the reference's `nimbus_infer_rs::sampler`
 * module (exported at src/lib.rs:20) and cites it.  The reference has no FFI
 * of its own; the Rust binding a maintainer would add (`extern "C"` block +
 * build.rs running hipcc) is shown in INTEGRATION.md.
 *
 * Conventions
 *   - Plain C types, caller-owned device buffers, no torch/HIP types in the
 *     signatures (streams travel as `void*` = hipStream_t).
 *   - Return 0 on success, a negative NIS_E* on an argument error (checked
 *     on the host before any launch), a positive hipError_t on a runtime
 *     error.  No C++ exception crosses the ABI.
 *   - One context = one device + one stream; a context is not thread-safe.
 *   - Batched calls are asynchronous on the context stream; nis_sync() or
 *     the caller's own stream synchronisation orders them.
 */
#ifndef NIMBUS_SAMPLER_H
#define NIMBUS_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NIS_ABI_VERSION 1

/* Status codes (negative: argument errors detected before launch). */
#define NIS_OK 0
#define NIS_EINVAL (-1)   /* null pointer, B<=0, V<=0, ld<V, reserved != 0 */
#define NIS_ERANGE (-2)   /* V or B beyond the supported maximum */
#define NIS_EALIGN (-3)   /* logits pointer not 4-byte aligned */
#define NIS_ENODEV (-4)   /* no HIP device / bad device ordinal */

/* Largest supported vocabulary (the penalty bitmap lives in LDS). */
#define NIS_MAX_V (1 << 20)
#define NIS_MAX_B (1 << 24)
/* Largest hidden size accepted by nis_lm_head_logits. */
#define NIS_MAX_H (1 << 20)

/* Sampling knobs of SamplingParams (sampler.rs:7-15), same f32 types:
 * temperature (sampler.rs:9; greedy iff <= 0, sampler.rs:32-34), top_k
 * (sampler.rs:10, usize, 0 disables), top_p (sampler.rs:11, >= 1 disables),
 * repetition_penalty (sampler.rs:12, 1.0 disables).  `seed`,
 * `max_new_tokens` and `stop_tokens` belong to the caller's decode loop
 * (engine.rs:266,271,285) and do not cross this boundary. */
typedef struct nis_params {
    float temperature;
    float top_p;
    float repetition_penalty;
    uint32_t reserved; /* must be 0 */
    uint64_t top_k;
} nis_params;

/* Which branch of sample() (sampler.rs:163-217) produced a row's token. */
#define NIS_PATH_GREEDY 1        /* temperature <= 0, sampler.rs:172-181 */
#define NIS_PATH_NONFINITE_MAX 2 /* filtered max not finite, sampler.rs:192-200 */
#define NIS_PATH_BAD_TOTAL 3     /* NaN / non-positive total, sampler.rs:206-208 */
#define NIS_PATH_DRAW 4          /* inverse-CDF draw, sampler.rs:209-214 */
#define NIS_PATH_FALLTHROUGH 5   /* walk overshoot returns V-1, sampler.rs:216 */

/* Optional per-row diagnostics (pass NULL to skip). */
typedef struct nis_row_stats {
    double max_w;   /* max of the filtered, temperature-scaled logits */
    double z_kept;  /* sum of exp(w - max_w) over kept tokens (`total`, sampler.rs:201-205) */
    double z_all;   /* same sum before top-p (top-p `sum`, sampler.rs:143); 0 if top-p inactive */
    double u;       /* next_f64() drawn (sampler.rs:209); -1 when the RNG was not advanced */
    double prob;    /* exp(w_token - max_w) / z_kept for a drawn token, else 0 */
    uint64_t kept;  /* tokens surviving top-k / top-p; counted on the DRAW and
                       FALLTHROUGH paths, 0 on the others */
    uint32_t path;  /* NIS_PATH_* */
    uint32_t token;
    uint32_t kernel;/* 1 = a row kernel (sparse, dense, resident, long-row), 2 = general path */
    uint32_t reject;/* NIS_REJECT_*: kernel 2 -> why the row kernel handed the row on
                       (SHAPE: no row kernel takes it); kernel 1 -> 0, or for a long
                       top-p row, why the single-read path handed it to the
                       long-row method that answered it */
} nis_row_stats;

/* nis_row_stats.reject: a row kernel declines a row it cannot prove exact
 * and the general path recomputes it; the result is the same either way. */
#define NIS_REJECT_NONE 0
#define NIS_REJECT_SHAPE 1      /* V out of range, per-row penalty, top-k, top-p <= 0 */
#define NIS_REJECT_NONFINITE 2  /* NaN / inf / empty row or exponent range */
#define NIS_REJECT_WINDOW 3     /* the estimated cutoff window missed the cutoff */
#define NIS_REJECT_CAPACITY 4   /* candidate list or cutoff bucket over capacity */
#define NIS_REJECT_BUCKET 5     /* cutoff bucket membership did not match its histogram,
                                   or the cutoff buckets hold more members than one
                                   wave ranks */

typedef struct nis_ctx nis_ctx;

/* Create a context on `device` with its own default-priority stream. */
int nis_ctx_create(int device, nis_ctx** out);
/* Destroy a context (synchronises its stream first). */
int nis_ctx_destroy(nis_ctx* ctx);
/* Launch on a caller stream (hipStream_t as void*, NULL = legacy default
 * stream) instead of the context's own; the caller keeps ownership. */
int nis_ctx_set_stream(nis_ctx* ctx, void* stream);
void* nis_ctx_get_stream(const nis_ctx* ctx);
/* Message of the last error recorded on `ctx` ("" if none). */
const char* nis_last_error(const nis_ctx* ctx);
/* Static text for a status code. */
const char* nis_status_string(int status);

/* Rng::new (sampler.rs:46-56): SplitMix64-seeded xoshiro256++ state. */
void nis_rng_seed(uint64_t seed, uint64_t state_out[4]);
/* Rng::next_u64 (sampler.rs:58-72) on a host-held state. */
uint64_t nis_rng_next_u64(uint64_t state[4]);
/* Rng::next_f64 (sampler.rs:75-77) on a host-held state. */
double nis_rng_next_f64(uint64_t state[4]);
/* Rng::new for B rows on the device: d_states[4*b..4*b+3] = Rng::new(d_seeds[b]). */
int nis_rng_seed_batch(nis_ctx* ctx, const uint64_t* d_seeds, int32_t B, uint64_t* d_states);

/* Batched sample() (sampler.rs:163-217) over row-major fp32 logits
 * [B, ld] in device memory, ld >= V.  Row b uses and advances the
 * xoshiro256++ state d_rng_state[4*b..4*b+3] exactly as the reference
 * advances `rng` (one next_u64 iff the row reaches sampler.rs:209).
 * Repetition penalty (sampler.rs:83-101) reads the CSR list
 * d_gen_ids[d_gen_offsets[b] .. d_gen_offsets[b+1]) (both may be NULL when
 * params->repetition_penalty == 1).  Writes d_tokens[b] and, if non-NULL,
 * d_stats[b].  Asynchronous on the context stream. */
int nis_sample_batch(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     const nis_params* params, uint64_t* d_rng_state,
                     const uint32_t* d_gen_ids, const int64_t* d_gen_offsets,
                     uint32_t* d_tokens, nis_row_stats* d_stats);

/* One step of a device-resident batched decode loop: the decode loop of
 * Engine::generate_ids (engine.rs:279-287) for B sequences at once, with the
 * model step left to the caller.  For every sequence b with d_done[b] == 0:
 *   token = sample(logits row b, params, history b, rng b)   (engine.rs:280)
 *   history b gets the token                                  (engine.rs:281)
 *   done when the token is one of the n_stop ids d_stop_ids, or the sequence
 *   has produced d_max_new[b] tokens                          (engine.rs:285)
 * History b is d_gen_ids[b*gen_cap .. b*gen_cap + d_gen_len[b]) and doubles
 * as the repetition-penalty list (the reference penalizes `generated`, not
 * the prompt); a full history (gen_len == gen_cap) also ends the sequence.
 * Sequences already done are skipped: no token written, RNG not advanced.
 * The caller starts with gen_len = 0 and done[b] = (max_new[b] <= 0), where
 * max_new[b] = min(max_new_tokens, max_seq_len - prompt length)
 * (engine.rs:265-266).  Same logits / params / RNG / stats contract as
 * nis_sample_batch.  Asynchronous on the context stream. */
int nis_decode_step(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                    const nis_params* params, uint64_t* d_rng_state, uint32_t* d_gen_ids,
                    int64_t gen_cap, int32_t* d_gen_len, const int32_t* d_max_new,
                    const uint32_t* d_stop_ids, int32_t n_stop, uint8_t* d_done,
                    uint32_t* d_tokens, nis_row_stats* d_stats);

/* Batched greedy: first index of the row maximum (sampler.rs:172-181);
 * same as nis_sample_batch with temperature 0 and no penalty. */
int nis_argmax_batch(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     uint32_t* d_tokens);

/* apply_repetition_penalty (sampler.rs:83-101) on a device f64 row:
 * d_logits[id] /= penalty if > 0 else *= penalty, once per distinct id < V. */
int nis_apply_repetition_penalty(nis_ctx* ctx, double* d_logits, int64_t V,
                                 const uint32_t* d_generated, int64_t n_generated,
                                 float penalty);

/* Single-row drop-in for sample(logits, params, generated, rng)
 * (sampler.rs:163-168): host logits and history are staged to the device
 * through a context-owned workspace, the HIP sampler runs, and the token and
 * advanced RNG state come back.  Synchronous. */
int nis_sample_one(nis_ctx* ctx, const float* h_logits, int64_t V, const nis_params* params,
                   const uint32_t* h_generated, int64_t n_generated, uint64_t state_inout[4],
                   uint32_t* token_out);

/* Allocation-free nis_sample_one.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, result and errors as nis_sample_one, but the row is staged
 * through a fixed static device array (NIS_NOALLOC_MAX_V logits and
 * NIS_NOALLOC_MAX_GEN history ids, about 1.25 MiB, held by each GPU the
 * library runs on until the process ends) instead of a context workspace:
 * it calls no hipMalloc / hipFree.  Larger V or histories return
 * NIS_ERANGE.  All calls on one GPU share that array, so calls that overlap
 * on one GPU (two threads, two contexts) race; serialize them. */
#define NIS_NOALLOC_MAX_V (1 << 18)
#define NIS_NOALLOC_MAX_GEN (1 << 16)
int nis_sample_one_noalloc(nis_ctx* ctx, const float* h_logits, int64_t V,
                           const nis_params* params, const uint32_t* h_generated,
                           int64_t n_generated, uint64_t state_inout[4], uint32_t* token_out);

/* LM-head weight formats (quant.rs:13-25): dense f32 rows; int8 codes stored
 * as value + 128 in bytes; int4 codes stored as value + 8, two per byte, low
 * nibble first over the global index row * H + k. */
#define NIS_W_F32 0
#define NIS_W_INT8 8
#define NIS_W_INT4 4

typedef struct nis_weights {
    int32_t format;         /* NIS_W_F32, NIS_W_INT8 or NIS_W_INT4 */
    int32_t group_size;     /* 0: one scale per row; else one per group_size input channels */
    const void* d_data;     /* [V][H] f32 / u8, or ceil(V*H/2) packed bytes */
    const float* d_scales;  /* [V] or [V][H/group_size]; unused for f32 */
} nis_weights;

/* The logits producer before sampling: d_logits[b*ld + v] = dot(d_hidden[b*ldh ..], W[v])
 * for B last-hidden rows, i.e. Model::logits_last (model.rs:317-325) through
 * Mat::gemv_into (model.rs:65-86) on a dense row (simd.rs:22) or
 * QuantMatrix::dot_rows_into (quant.rs:121-161): a per-row scale multiplies
 * the row's dot product, group scales each group's.  Sums are f32 in the
 * library's own order (the reference's is its SIMD lane order): each logit is
 * within the f32 error bound of a length-H sum of its exact value.  int4
 * needs an even H and group size (the reference's reader assumes even nibble
 * offsets).  Asynchronous on the context stream; the output feeds
 * nis_sample_batch / nis_decode_step on the same stream. */
int nis_lm_head_logits(nis_ctx* ctx, const float* d_hidden, int64_t ldh, int32_t B, int32_t H,
                       const nis_weights* w, int64_t V, float* d_logits, int64_t ld);

/* Greedy decoding of one hidden row: *d_token = the first index of the
 * maximum of the logits nis_lm_head_logits would produce for B = 1
 * (Model::logits_last, model.rs:317-325, then sample()'s greedy branch,
 * sampler.rs:172-181: a NaN at index 0 gives 0, other NaNs never win).  The
 * one-row GEMV keeps each workgroup's first maximum in its epilogue and one
 * small workgroup reduces those, so the logits are not read again.  d_logits
 * [V] may be null (then they are not written).  No counterpart in the
 * reference, which has no fused form: it is nis_lm_head_logits followed by
 * nis_argmax_batch in one pass, for a decode loop that wants the token only.
 * The first call allocates the context's key buffer (512 KiB); a shape the
 * one-row kernel does not take runs those two calls instead (with a context-
 * owned logits buffer when d_logits is null).  Asynchronous on the context
 * stream. */
int nis_lm_head_greedy(nis_ctx* ctx, const float* d_hidden, int32_t H, const nis_weights* w, int64_t V,
                       float* d_logits, uint32_t* d_token);

/* Measurement only: the bandwidth floor of the sparse row kernel.  One
 * 1024-lane workgroup per row reads it with that kernel's layout and load
 * pipeline and computes only each row's max and sum of 2^(x c - R)
 * (d_out[2 b] = max, d_out[2 b + 1] = the sum at R = ceil(max c),
 * c = log2(e) / max(T, 1e-6)); it samples nothing.  No counterpart in the
 * reference: bench.py --floor times it beside the sampler, so that the
 * sampler's roofline fraction has a measured ceiling.  256 <= V <= 53245.
 * Asynchronous on the context stream. */
int nis_stream_floor(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     float temperature, float* d_out);

/* Measurement only: the floor of splitting rows over workgroups.  Row b is
 * read by S workgroups of 256 lanes (a slice of the row's float4 slots
 * each, 1 <= S <= 64, at most 4096 slots per slice); each of their waves
 * writes its slice's max and sum of 2^(x c - R_w) to d_part (B * S * 4
 * records of 16 bytes, 16-byte aligned), and a second launch merges a row's
 * records into d_out as nis_stream_floor does.  No counterpart in the
 * reference: bench.py --floor --split S times it, the least any sampler
 * that splits rows pays per merge.  Asynchronous on the context stream. */
int nis_stream_floor_split(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                           float temperature, int32_t S, void* d_part, float* d_out);

/* Wait for all work queued on the context stream. */
int nis_sync(nis_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif /* NIMBUS_SAMPLER_H */
