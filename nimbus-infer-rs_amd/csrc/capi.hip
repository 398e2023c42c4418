// capi.hip — implementation of the C ABI in include/nimbus_sampler.h.
//
// Host-side argument checking happens before any launch; device work is
// asynchronous on the context stream.  There is no CPU fallback: every
// sampling entry point launches the gfx950 kernels or returns an error.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "kernels.h"
#include "floor_path.h"
#include "lm_head.h"

// 16-row hidden tiles per matrix-core wave when B > 16 (4 or 2)
#ifndef NIS_LH_NB
#define NIS_LH_NB 4
#endif
// parts of h summed by separate waves at 4 tiles per wave (1, 2 or 4)
#ifndef NIS_LH_KS
#define NIS_LH_KS 2
#endif
#include "nimbus_sampler.h"
#include "rng.h"

struct nis_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    // staging for nis_sample_one
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // nis_lm_head_greedy: the workgroup keys, and logits when the caller
    // passes none to a call that needs them
    unsigned long long* gpart = nullptr;
    float* glogits = nullptr;
    int64_t glogits_n = 0;
};

namespace {

// Staging area of nis_sample_one_noalloc: RNG state, token, history offsets,
// history and logits of one row, laid out by noalloc_layout().  Each device
// holds its own copy for the life of the process; host code reaches it only
// through the per-device address that hipGetSymbolAddress returns.
constexpr size_t kNoAllocStateOff = 0;
constexpr size_t kNoAllocTokOff = 256;
constexpr size_t kNoAllocGoffOff = 512;
constexpr size_t kNoAllocGenOff = 1024;
constexpr size_t kNoAllocLogitsOff = kNoAllocGenOff + (size_t)NIS_NOALLOC_MAX_GEN * 4;
constexpr size_t kNoAllocBytes = kNoAllocLogitsOff + (size_t)NIS_NOALLOC_MAX_V * 4;
static_assert(kNoAllocLogitsOff % 256 == 0, "logits staging must stay 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `dev`, which must be the current device.
// Looked up once per device (at nis_ctx_create, or on the first
// nis_sample_one_noalloc call if that lookup failed) and kept.
hipError_t scratch_on_device(int dev, void** out) {
    *out = nullptr;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!ptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

// Make `dev` current for the duration of a call and restore the caller's.
struct DeviceGuard {
    int prev = -1;
    hipError_t status = hipSuccess;
    explicit DeviceGuard(int dev) {
        status = hipGetDevice(&prev);
        if (status == hipSuccess && prev != dev) status = hipSetDevice(dev);
        else if (status == hipSuccess) prev = -1;
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

int fail(nis_ctx* ctx, int code, const char* msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int hip_fail(nis_ctx* ctx, hipError_t e, const char* where) {
    if (ctx) {
        ctx->err = where;
        ctx->err += ": ";
        ctx->err += hipGetErrorString(e);
    }
    return (int)e;
}

int check_batch_args(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     const nis_params* p, const uint64_t* d_rng, const uint32_t* d_gen_ids,
                     const int64_t* d_gen_off, const uint32_t* d_tokens) {
    if (!ctx) return NIS_EINVAL;
    if (!d_logits || !p || !d_tokens) return fail(ctx, NIS_EINVAL, "null pointer argument");
    if (B <= 0) return fail(ctx, NIS_EINVAL, "B must be positive");
    if (V <= 0) return fail(ctx, NIS_EINVAL, "V must be positive");
    if (ld < V) return fail(ctx, NIS_EINVAL, "ld must be >= V");
    if (V > NIS_MAX_V) return fail(ctx, NIS_ERANGE, "V exceeds NIS_MAX_V");
    if (B > NIS_MAX_B) return fail(ctx, NIS_ERANGE, "B exceeds NIS_MAX_B");
    if (p->reserved != 0) return fail(ctx, NIS_EINVAL, "nis_params.reserved must be 0");
    if (((uintptr_t)d_logits & 3u) != 0) return fail(ctx, NIS_EALIGN, "logits not 4-byte aligned");
    if (!(p->temperature <= 0.0f) && !d_rng)
        return fail(ctx, NIS_EINVAL, "rng state required unless temperature <= 0");
    if ((d_gen_ids == nullptr) != (d_gen_off == nullptr))
        return fail(ctx, NIS_EINVAL, "gen_ids and gen_offsets must both be set or both NULL");
    return NIS_OK;
}

nis::RowArgs row_args(const float* d_logits, int64_t ld, int64_t V, const nis_params* params,
                      uint64_t* d_rng_state, uint32_t* d_tokens, nis_row_stats* d_stats) {
    nis::RowArgs a;
    a.logits = d_logits;
    a.ld = ld;
    a.V = V;
    a.temperature = params->temperature;
    a.top_p = params->top_p;
    a.penalty = params->repetition_penalty;
    a.top_k = params->top_k;
    a.rng = d_rng_state;
    a.gen_ids = nullptr;
    a.gen_off = nullptr;
    a.gen_len = nullptr;
    a.gen_cap = 0;
    a.done = nullptr;
    a.gen_out = nullptr;
    a.max_new = nullptr;
    a.stop = nullptr;
    a.n_stop = 0;
    a.tokens = d_tokens;
    a.stats = d_stats;
    return a;
}

// One kernel per launch, by the launch's parameters (every kernel computes
// every row exactly; this only picks the faster):
//   - greedy (T <= 0), 256 <= V <= 53245: the resident kernel's argmax;
//   - top-p off (>= 1), no top-k: the resident kernel's all-kept walk;
//   - 0.95 <= top-p < 1, no top-k: the 1024-lane dense kernel (a nucleus of
//     any size: one exact histogram of the whole row built in the stream),
//     or its penalty variant for a launch with a penalty history;
//   - 0 < top-p < 0.95, no top-k: the 1024-lane sparse kernel (few kept
//     tokens, listed against a sampled threshold);
//   - 0 < top-k < V with any top-p > 0 and no penalty history: the sparse
//     kernel's top-k form (the k-th largest found by count in the same
//     histograms, top-p searched on the top-k mass);
//   - 53245 < V <= 262141, 0 < top-p < 0.95, no top-k, no penalty history:
//     the 1024-lane long sparse kernel (the row read once, its candidates
//     listed in LDS against a pooled sampled threshold; a declined row runs
//     the long-row method, then the general path, inside the same kernel);
//   - other rows with V > 53245, no top-k: the 512-lane long-row kernel
//     (greedy, top-p off or top-p, the row read again from cache after its
//     stream), then the general path on the rows it declined;
//   - anything else (V < 256, top-p <= 0, top-k with a penalty history or
//     past 53245, a penalty history on rows longer than the registers hold):
//     the 512-lane general kernel.
// A row one of these kernels cannot prove (non-finite values, capacity,
// exact-tie overflow, a history past the bitmaps) runs the general path
// inside whichever kernel was launched.
int launch_rows(nis_ctx* ctx, const nis::RowArgs& a, int32_t B) {
    const bool res_shape = a.V >= 256 && a.V <= nis::kRMaxV;
    const bool no_topk = a.top_k == 0 || a.top_k >= (uint64_t)a.V;
    if (res_shape && a.temperature <= 0.0f) {
        if (a.penalty != 1.0f && a.gen_ids != nullptr)  // the penalty applied in registers
            hipLaunchKernelGGL(nis::sample_rows_resident_kernel<nis::kResGreedyPen>, dim3((unsigned)B),
                               dim3(nis::kRB), 0, ctx->stream, a);
        else
            hipLaunchKernelGGL(nis::sample_rows_resident_kernel<nis::kResGreedy>, dim3((unsigned)B),
                               dim3(nis::kRB), 0, ctx->stream, a);
    } else if (res_shape && a.temperature > 0.0f && no_topk && a.top_p >= 1.0f) {
        if (a.penalty != 1.0f && a.gen_ids != nullptr)  // the penalty applied in registers
            hipLaunchKernelGGL(nis::sample_rows_resident_kernel<nis::kResAllPen>, dim3((unsigned)B),
                               dim3(nis::kRB), 0, ctx->stream, a);
        else
            hipLaunchKernelGGL(nis::sample_rows_resident_kernel<nis::kResAll>, dim3((unsigned)B),
                               dim3(nis::kRB), 0, ctx->stream, a);
    } else if (res_shape && a.temperature > 0.0f && no_topk && a.top_p >= 0.95f && a.top_p < 1.0f) {
        if (a.penalty != 1.0f && a.gen_ids != nullptr)  // the penalty applied in registers
            hipLaunchKernelGGL(nis::sample_rows_dense_pen_kernel, dim3((unsigned)B), dim3(nis::kDB), 0,
                               ctx->stream, a);
        else
            hipLaunchKernelGGL(nis::sample_rows_dense_kernel, dim3((unsigned)B), dim3(nis::kDB), 0,
                               ctx->stream, a);
    } else if (a.V >= 256 && a.V <= nis::kSMaxV && a.temperature > 0.0f && a.top_p > 0.0f &&
               a.top_p < 0.95f && no_topk && (a.penalty == 1.0f || a.gen_ids == nullptr)) {
        hipLaunchKernelGGL(nis::sample_rows_sparse_kernel, dim3((unsigned)B), dim3(nis::kSB), 0,
                           ctx->stream, a);
    } else if (a.V >= 256 && a.V <= nis::kSMaxV && a.temperature > 0.0f && a.top_p > 0.0f &&
               a.top_p < 0.95f && no_topk) {
        // a repetition-penalty history: applied inside the sparse path; the
        // rows it declines (long histories) finish on the dense path
        hipLaunchKernelGGL(nis::sample_rows_sparse_pen_kernel, dim3((unsigned)B), dim3(nis::kSB), 0,
                           ctx->stream, a);
        hipLaunchKernelGGL(nis::sample_rows_dense_pending_kernel, dim3((unsigned)B), dim3(nis::kDB), 0,
                           ctx->stream, a);
    } else if (a.V >= 256 && a.V <= nis::kSMaxV && a.temperature > 0.0f && a.top_p > 0.0f && !no_topk &&
               (a.penalty == 1.0f || a.gen_ids == nullptr)) {
        // top-k (with top-p at any p > 0): found by count in the sparse path
        hipLaunchKernelGGL(nis::sample_rows_sparse_topk_kernel, dim3((unsigned)B), dim3(nis::kSB), 0,
                           ctx->stream, a);
    } else if (a.V > nis::kSMaxV && a.V <= nis::kLSMaxV && a.temperature > 0.0f && a.top_p > 0.0f &&
               a.top_p < 0.95f && no_topk && (a.penalty == 1.0f || a.gen_ids == nullptr)) {
        // long top-p rows, read once (declined rows finish inside the kernel)
        hipLaunchKernelGGL(nis::sample_rows_long_sparse_kernel, dim3((unsigned)B), dim3(nis::kLSB), 0,
                           ctx->stream, a);
    } else if (a.V > nis::kDMaxV &&
               (a.temperature <= 0.0f ||
                (no_topk && (a.penalty == 1.0f || a.gen_ids == nullptr || a.top_p >= 1.0f)))) {
        // (greedy and top-p off take a penalty history on the long-row kernel)
        if (a.temperature <= 0.0f)
            hipLaunchKernelGGL(nis::sample_rows_long_kernel<nis::kLongGreedy>, dim3((unsigned)B),
                               dim3(nis::kLB), 0, ctx->stream, a);
        else if (a.top_p >= 1.0f)
            hipLaunchKernelGGL(nis::sample_rows_long_kernel<nis::kLongAll>, dim3((unsigned)B),
                               dim3(nis::kLB), 0, ctx->stream, a);
        else
            hipLaunchKernelGGL(nis::sample_rows_long_kernel<nis::kLongTopP>, dim3((unsigned)B),
                               dim3(nis::kLB), 0, ctx->stream, a);
        // the rows it declined (penalty history past its reach, non-finite,
        // exact-tie overflow, a top-p row's span)
        hipLaunchKernelGGL(nis::sample_rows_pending_kernel, dim3((unsigned)std::min(B, 256)),
                           dim3(nis::kBlock), 0, ctx->stream, a, B);
    } else {
        hipLaunchKernelGGL(nis::sample_rows_kernel, dim3((unsigned)B), dim3(nis::kBlock), 0,
                           ctx->stream, a);
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "sample kernel launch");
}

template <int FMT, bool VEC, bool GROUPED>
void launch_lm_head_t(const nis::LmHeadArgs& a, int nb, dim3 grid, dim3 block, hipStream_t st) {
    if (nb == 4)  // (h split in NIS_LH_KS parts: see lm_head_kernel)
        hipLaunchKernelGGL((nis::lm_head_kernel<FMT, VEC, GROUPED, 4, NIS_LH_KS>), grid, block, 0, st, a);
    else if (nb == 2)
        hipLaunchKernelGGL((nis::lm_head_kernel<FMT, VEC, GROUPED, 2, 1>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((nis::lm_head_kernel<FMT, VEC, GROUPED, 1, 1>), grid, block, 0, st, a);
}

template <int FMT>
void launch_lm_head_f(const nis::LmHeadArgs& a, bool vec, bool grouped, int nb, dim3 grid,
                      dim3 block, hipStream_t st) {
    if (vec && grouped) launch_lm_head_t<FMT, true, true>(a, nb, grid, block, st);
    else if (vec) launch_lm_head_t<FMT, true, false>(a, nb, grid, block, st);
    else if (grouped) launch_lm_head_t<FMT, false, true>(a, nb, grid, block, st);
    else launch_lm_head_t<FMT, false, false>(a, nb, grid, block, st);
}

// The one-hidden-row GEMV (lm_head_row_kernel) when its shape holds: whole
// runs per row (H % R == 0), one scale per run, aligned operands and at most
// 4 runs per lane with 16 or 64 lanes per row (3 when they suffice, which
// keeps fewer hidden values in registers).  Returns false to leave the call
// to the matrix-core kernel.
// nis_lm_head_greedy: workgroup keys kept per context (a fused launch of more
// workgroups takes the two-launch form instead)
constexpr int64_t kGreedyMaxBlocks = 1 << 16;

template <int FMT, bool GREEDY, int KM>
void launch_lm_head_row_km(const nis::LmHeadArgs& a, bool grouped, dim3 grid, hipStream_t st, int log2L,
                           int runs) {
    if (grouped)
        hipLaunchKernelGGL((nis::lm_head_row_kernel<FMT, true, GREEDY, KM>), grid, dim3(256), 0, st, a, log2L,
                           runs);
    else
        hipLaunchKernelGGL((nis::lm_head_row_kernel<FMT, false, GREEDY, KM>), grid, dim3(256), 0, st, a, log2L,
                           runs);
}

template <int FMT, bool GREEDY = false>
bool launch_lm_head_row(const nis::LmHeadArgs& a, bool grouped, uintptr_t wp, hipStream_t st,
                        int64_t* blocks = nullptr) {
    constexpr int R = nis::LhRowCfg<FMT>::R;
    if (a.H % R != 0 || (wp & 15u) != 0 || ((uintptr_t)a.x & 15u) != 0) return false;
    if (grouped && a.group % R != 0) return false;
    const int runs = a.H / R;
    int log2L, km;
    if ((runs + 15) / 16 <= 4) log2L = 4, km = (runs + 15) / 16 <= 3 ? 3 : 4;
    else if ((runs + 63) / 64 <= 4) log2L = 6, km = (runs + 63) / 64 <= 3 ? 3 : 4;
    else return false;
    const int64_t rows_per_wave = (int64_t)(64 >> log2L) * nis::LhRowCfg<FMT>::ITER;
    const int64_t waves = (a.V + rows_per_wave - 1) / rows_per_wave;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (blocks) *blocks = (int64_t)grid.x;
    if (GREEDY && (int64_t)grid.x > kGreedyMaxBlocks) return false;
    if (km == 3) launch_lm_head_row_km<FMT, GREEDY, 3>(a, grouped, grid, st, log2L, runs);
    else launch_lm_head_row_km<FMT, GREEDY, 4>(a, grouped, grid, st, log2L, runs);
    return true;
}

// Argument checks of the LM-head entry points, and their kernel arguments.
int lm_head_setup(nis_ctx* ctx, const float* d_hidden, int64_t ldh, int32_t B, int32_t H,
                  const nis_weights* w, int64_t V, float* d_logits, int64_t ld, bool logits_optional,
                  nis::LmHeadArgs& a, bool& grouped, bool& vec, uintptr_t& wp) {
    if (!ctx) return NIS_EINVAL;
    if (!d_hidden || !w || (!d_logits && !logits_optional) || !w->d_data)
        return fail(ctx, NIS_EINVAL, "null pointer argument");
    if (B <= 0 || H <= 0 || V <= 0) return fail(ctx, NIS_EINVAL, "B, H and V must be positive");
    if (ldh < H || ld < V) return fail(ctx, NIS_EINVAL, "ldh must be >= H and ld >= V");
    if (B > NIS_MAX_B || V > NIS_MAX_V || H > NIS_MAX_H) return fail(ctx, NIS_ERANGE, "B, H or V too large");
    const int fmt = w->format;
    if (fmt != NIS_W_F32 && fmt != NIS_W_INT8 && fmt != NIS_W_INT4)
        return fail(ctx, NIS_EINVAL, "unknown weight format");
    const int32_t g = w->group_size;
    if (fmt == NIS_W_F32) {
        if (g != 0) return fail(ctx, NIS_EINVAL, "f32 weights take no group size");
    } else {
        if (!w->d_scales) return fail(ctx, NIS_EINVAL, "quantized weights need scales");
        if (g < 0 || (g > 0 && H % g != 0)) return fail(ctx, NIS_EINVAL, "group size must divide H");
        // the reference's int4 row / group reader starts at a low nibble
        // (quant.rs:130-133, 150-152), which is its packing only at even offsets
        if (fmt == NIS_W_INT4 && (H % 2 != 0 || g % 2 != 0))
            return fail(ctx, NIS_EINVAL, "int4 weights need an even H and group size");
    }
    if (((uintptr_t)d_hidden & 3u) || ((uintptr_t)d_logits & 3u) || ((uintptr_t)w->d_scales & 3u) ||
        (fmt == NIS_W_F32 && ((uintptr_t)w->d_data & 3u)))
        return fail(ctx, NIS_EALIGN, "hidden, logits, scales and f32 weights must be 4-byte aligned");

    a.x = d_hidden;
    a.ldx = ldh;
    a.B = B;
    a.H = H;
    a.w = w->d_data;
    a.scales = w->d_scales;
    a.group = g > 0 ? g : H;
    a.groups = H / a.group;
    // ceil(2^32 / group) fits 32 bits for group >= 2; group 1 is marked by 0
    a.gmagic = a.group == 1 ? 0u
                            : (uint32_t)((((uint64_t)1 << 32) + (uint64_t)a.group - 1) / (uint64_t)a.group);
    a.V = V;
    a.out = d_logits;
    a.ld = ld;
    a.part = nullptr;
    grouped = fmt != NIS_W_F32 && a.groups > 1;
    wp = (uintptr_t)w->d_data;
    vec = H % 4 == 0 && ldh % 4 == 0 && ((uintptr_t)d_hidden & 15u) == 0 &&
          (!grouped || a.group % 4 == 0) &&
          ((fmt == NIS_W_F32 && (wp & 15u) == 0) || (fmt == NIS_W_INT8 && (wp & 3u) == 0) ||
           (fmt == NIS_W_INT4 && (wp & 1u) == 0));
    return NIS_OK;
}

}  // namespace

extern "C" {

const char* nis_status_string(int status) {
    switch (status) {
        case NIS_OK: return "ok";
        case NIS_EINVAL: return "invalid argument";
        case NIS_ERANGE: return "size out of range";
        case NIS_EALIGN: return "misaligned pointer";
        case NIS_ENODEV: return "no such HIP device";
        default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
    }
}

int nis_ctx_create(int device, nis_ctx** out) {
    if (!out) return NIS_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return NIS_ENODEV;
    nis_ctx* ctx = new (std::nothrow) nis_ctx();
    if (!ctx) return (int)hipErrorOutOfMemory;
    ctx->device = device;
    DeviceGuard g(device);
    if (g.status != hipSuccess) {
        delete ctx;
        return (int)g.status;
    }
    hipError_t e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return (int)e;
    }
    ctx->stream = ctx->own_stream;
    void* scr = nullptr;
    (void)scratch_on_device(device, &scr);  // retried by nis_sample_one_noalloc on failure
    *out = ctx;
    return NIS_OK;
}

int nis_ctx_destroy(nis_ctx* ctx) {
    if (!ctx) return NIS_EINVAL;
    DeviceGuard g(ctx->device);
    int rc = NIS_OK;
    if (ctx->own_stream) {
        hipError_t e = hipStreamSynchronize(ctx->own_stream);
        if (e != hipSuccess) rc = (int)e;
        (void)hipStreamDestroy(ctx->own_stream);
    }
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->gpart) (void)hipFree(ctx->gpart);
    if (ctx->glogits) (void)hipFree(ctx->glogits);
    delete ctx;
    return rc;
}

int nis_ctx_set_stream(nis_ctx* ctx, void* stream) {
    if (!ctx) return NIS_EINVAL;
    ctx->stream = (hipStream_t)stream;
    return NIS_OK;
}

void* nis_ctx_get_stream(const nis_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

const char* nis_last_error(const nis_ctx* ctx) { return ctx ? ctx->err.c_str() : ""; }

void nis_rng_seed(uint64_t seed, uint64_t state_out[4]) {
    if (state_out) nis::rng_seed(seed, state_out);
}

uint64_t nis_rng_next_u64(uint64_t state[4]) { return state ? nis::rng_next_u64(state) : 0; }

double nis_rng_next_f64(uint64_t state[4]) { return state ? nis::rng_next_f64(state) : 0.0; }

int nis_rng_seed_batch(nis_ctx* ctx, const uint64_t* d_seeds, int32_t B, uint64_t* d_states) {
    if (!ctx) return NIS_EINVAL;
    if (!d_seeds || !d_states) return fail(ctx, NIS_EINVAL, "null pointer argument");
    if (B <= 0 || B > NIS_MAX_B) return fail(ctx, B <= 0 ? NIS_EINVAL : NIS_ERANGE, "bad B");
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");
    const int threads = 256;
    hipLaunchKernelGGL(nis::rng_seed_kernel, dim3((B + threads - 1) / threads), dim3(threads), 0,
                       ctx->stream, d_seeds, B, d_states);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "rng_seed_kernel launch");
}

int nis_sample_batch(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     const nis_params* params, uint64_t* d_rng_state, const uint32_t* d_gen_ids,
                     const int64_t* d_gen_offsets, uint32_t* d_tokens, nis_row_stats* d_stats) {
    int rc = check_batch_args(ctx, d_logits, ld, B, V, params, d_rng_state, d_gen_ids,
                              d_gen_offsets, d_tokens);
    if (rc != NIS_OK) return rc;
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");
    nis::RowArgs a = row_args(d_logits, ld, V, params, d_rng_state, d_tokens, d_stats);
    a.gen_ids = d_gen_ids;
    a.gen_off = d_gen_offsets;
    return launch_rows(ctx, a, B);
}

int nis_decode_step(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                    const nis_params* params, uint64_t* d_rng_state, uint32_t* d_gen_ids,
                    int64_t gen_cap, int32_t* d_gen_len, const int32_t* d_max_new,
                    const uint32_t* d_stop_ids, int32_t n_stop, uint8_t* d_done,
                    uint32_t* d_tokens, nis_row_stats* d_stats) {
    int rc = check_batch_args(ctx, d_logits, ld, B, V, params, d_rng_state, nullptr, nullptr,
                              d_tokens);
    if (rc != NIS_OK) return rc;
    if (!d_gen_ids || !d_gen_len || !d_max_new || !d_done)
        return fail(ctx, NIS_EINVAL, "gen_ids, gen_len, max_new and done are required");
    if (gen_cap <= 0) return fail(ctx, NIS_EINVAL, "gen_cap must be positive");
    if (gen_cap > ((int64_t)1 << 31) - 1) return fail(ctx, NIS_ERANGE, "gen_cap exceeds INT32_MAX");
    if (n_stop < 0 || (n_stop > 0 && !d_stop_ids))
        return fail(ctx, NIS_EINVAL, "n_stop must be >= 0 with stop ids when positive");
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");
    nis::RowArgs a = row_args(d_logits, ld, V, params, d_rng_state, d_tokens, d_stats);
    a.gen_ids = d_gen_ids;
    a.gen_len = d_gen_len;
    a.gen_cap = gen_cap;
    a.done = d_done;
    a.gen_out = d_gen_ids;
    a.max_new = d_max_new;
    a.stop = d_stop_ids;
    a.n_stop = n_stop;
    return launch_rows(ctx, a, B);  // the row kernels append, stop and count in place
}

int nis_argmax_batch(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     uint32_t* d_tokens) {
    nis_params p;
    p.temperature = 0.0f;
    p.top_p = 1.0f;
    p.repetition_penalty = 1.0f;
    p.reserved = 0;
    p.top_k = 0;
    return nis_sample_batch(ctx, d_logits, ld, B, V, &p, nullptr, nullptr, nullptr, d_tokens,
                            nullptr);
}

int nis_apply_repetition_penalty(nis_ctx* ctx, double* d_logits, int64_t V,
                                 const uint32_t* d_generated, int64_t n_generated,
                                 float penalty) {
    if (!ctx) return NIS_EINVAL;
    if (!d_logits || (n_generated > 0 && !d_generated))
        return fail(ctx, NIS_EINVAL, "null pointer argument");
    if (V <= 0 || n_generated < 0) return fail(ctx, NIS_EINVAL, "bad size");
    if (V > NIS_MAX_V) return fail(ctx, NIS_ERANGE, "V exceeds NIS_MAX_V");
    if (penalty == 1.0f || n_generated == 0) return NIS_OK;  // sampler.rs:84-86
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");
    hipLaunchKernelGGL(nis::repetition_penalty_kernel, dim3(1), dim3(nis::kBlock), 0, ctx->stream,
                       d_logits, V, d_generated, n_generated, (double)penalty);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "penalty kernel launch");
}

int nis_lm_head_logits(nis_ctx* ctx, const float* d_hidden, int64_t ldh, int32_t B, int32_t H,
                       const nis_weights* w, int64_t V, float* d_logits, int64_t ld) {
    nis::LmHeadArgs a;
    bool grouped = false, vec = false;
    uintptr_t wp = 0;
    int rc = lm_head_setup(ctx, d_hidden, ldh, B, H, w, V, d_logits, ld, false, a, grouped, vec, wp);
    if (rc != NIS_OK) return rc;
    const int fmt = w->format;
    DeviceGuard dg(ctx->device);
    if (dg.status != hipSuccess) return hip_fail(ctx, dg.status, "hipSetDevice");
    if (B == 1 && fmt == NIS_W_F32) {
        if (launch_lm_head_row<nis::kLhF32>(a, false, wp, ctx->stream)) goto launched;
    } else if (B == 1 && fmt == NIS_W_INT8) {
        if (launch_lm_head_row<nis::kLhInt8>(a, grouped, wp, ctx->stream)) goto launched;
    } else if (B == 1) {
        if (launch_lm_head_row<nis::kLhInt4>(a, grouped, wp, ctx->stream)) goto launched;
    }
    {
    // a wave: 64 vocab rows x 16*nb hidden rows; workgroups of 1 wave for
    // small batches (spread over every CU), else 4 waves split along b first
    // (nb = 4: 4 / NIS_LH_KS tiles along b, each summed by NIS_LH_KS waves
    // over parts of h, whole 32-wide chunks)
    const int nb = B > 16 ? NIS_LH_NB : 1;
    const int64_t nbt = ((int64_t)B + 16 * nb - 1) / (16 * nb);
    const int ks = nb == 4 ? NIS_LH_KS : 1;
    a.wb = nb == 1 ? 1 : (nbt >= 4 / ks ? 4 / ks : (nbt >= 2 ? 2 : 1));
    a.wv = nb == 1 ? 1 : 4 / ks / a.wb;
    a.hs = ((H / ks + 31) / 32) * 32;
    dim3 grid((unsigned)((nbt + a.wb - 1) / a.wb), (unsigned)((V + 64 * a.wv - 1) / (64 * a.wv)));
    if (ks > 1) {  // 1-D, the vocab tiles rounded up to whole groups of 8 (see lm_head_kernel)
        a.gx = (int32_t)grid.x;
        grid = dim3((unsigned)(grid.x * ((grid.y + 7) / 8) * 8), 1u);
    }
    dim3 block((unsigned)(64 * a.wv * a.wb * ks));
    if (fmt == NIS_W_F32) launch_lm_head_f<nis::kLhF32>(a, vec, false, nb, grid, block, ctx->stream);
    else if (fmt == NIS_W_INT8) launch_lm_head_f<nis::kLhInt8>(a, vec, grouped, nb, grid, block, ctx->stream);
    else launch_lm_head_f<nis::kLhInt4>(a, vec, grouped, nb, grid, block, ctx->stream);
    }
launched:
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "lm_head kernel launch");
}

int nis_lm_head_greedy(nis_ctx* ctx, const float* d_hidden, int32_t H, const nis_weights* w, int64_t V,
                       float* d_logits, uint32_t* d_token) {
    if (!ctx) return NIS_EINVAL;
    if (!d_token) return fail(ctx, NIS_EINVAL, "null pointer argument");
    nis::LmHeadArgs a;
    bool grouped = false, vec = false;
    uintptr_t wp = 0;
    int rc = lm_head_setup(ctx, d_hidden, H, 1, H, w, V, d_logits, V, true, a, grouped, vec, wp);
    if (rc != NIS_OK) return rc;
    DeviceGuard dg(ctx->device);
    if (dg.status != hipSuccess) return hip_fail(ctx, dg.status, "hipSetDevice");
    if (!ctx->gpart) {  // once per context: the fused launch's workgroup keys
        hipError_t e = hipMalloc((void**)&ctx->gpart, (size_t)kGreedyMaxBlocks * sizeof(unsigned long long));
        if (e != hipSuccess) {
            ctx->gpart = nullptr;
            return hip_fail(ctx, e, "hipMalloc greedy keys");
        }
    }
    a.part = ctx->gpart;
    const int fmt = w->format;
    int64_t blocks = 0;
    bool fused = false;
    if (fmt == NIS_W_F32) fused = launch_lm_head_row<nis::kLhF32, true>(a, false, wp, ctx->stream, &blocks);
    else if (fmt == NIS_W_INT8) fused = launch_lm_head_row<nis::kLhInt8, true>(a, grouped, wp, ctx->stream, &blocks);
    else fused = launch_lm_head_row<nis::kLhInt4, true>(a, grouped, wp, ctx->stream, &blocks);
    if (fused) {
        hipLaunchKernelGGL(nis::lm_head_greedy_final_kernel, dim3(1), dim3(1024), 0, ctx->stream,
                           (const unsigned long long*)ctx->gpart, (int)blocks, d_token);
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "lm_head greedy launch");
    }
    // a shape the one-row kernel does not take: the logits, then the greedy
    // row kernel over them
    float* lg = d_logits;
    if (!lg) {
        if (ctx->glogits_n < V) {
            if (ctx->glogits) (void)hipFree(ctx->glogits);
            ctx->glogits_n = 0;
            hipError_t e = hipMalloc((void**)&ctx->glogits, (size_t)V * sizeof(float));
            if (e != hipSuccess) {
                ctx->glogits = nullptr;
                return hip_fail(ctx, e, "hipMalloc greedy logits");
            }
            ctx->glogits_n = V;
        }
        lg = ctx->glogits;
    }
    rc = nis_lm_head_logits(ctx, d_hidden, H, 1, H, w, V, lg, V);
    if (rc != NIS_OK) return rc;
    return nis_argmax_batch(ctx, lg, V, 1, V, d_token);
}

int nis_stream_floor(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                     float temperature, float* d_out) {
    if (!ctx) return NIS_EINVAL;
    if (!d_logits || !d_out) return fail(ctx, NIS_EINVAL, "null pointer argument");
    if (B <= 0 || V < 256 || V > nis::kSMaxV || ld < V)
        return fail(ctx, NIS_EINVAL, "B must be positive, 256 <= V <= 53245 and ld >= V");
    if (B > NIS_MAX_B) return fail(ctx, NIS_ERANGE, "B too large");
    if (((uintptr_t)d_logits & 3u) || ((uintptr_t)d_out & 3u))
        return fail(ctx, NIS_EALIGN, "logits and out must be 4-byte aligned");
    if (!(temperature > 0.0f)) return fail(ctx, NIS_EINVAL, "temperature must be positive");
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");
    const float c = (float)(1.4426950408889634 / fmax((double)temperature, 1e-6));
    hipLaunchKernelGGL(nis::stream_floor_kernel, dim3((unsigned)B), dim3(nis::kSB), 0, ctx->stream,
                       d_logits, ld, (int)V, c, d_out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "stream floor launch");
}

int nis_stream_floor_split(nis_ctx* ctx, const float* d_logits, int64_t ld, int32_t B, int64_t V,
                           float temperature, int32_t S, void* d_part, float* d_out) {
    if (!ctx) return NIS_EINVAL;
    if (!d_logits || !d_out || !d_part) return fail(ctx, NIS_EINVAL, "null pointer argument");
    if (B <= 0 || V < 256 || V > nis::kSMaxV || ld < V)
        return fail(ctx, NIS_EINVAL, "B must be positive, 256 <= V <= 53245 and ld >= V");
    if (B > NIS_MAX_B) return fail(ctx, NIS_ERANGE, "B too large");
    const int64_t nsl = (V + 3 + 3) / 4;  // slots touching a row (at most)
    if (S < 1 || S > 64 || (nsl + S - 1) / S > (int64_t)nis::kFPB * nis::kFPN)
        return fail(ctx, NIS_EINVAL, "S must be 1..64 with at most 4096 float4 slots per slice");
    if (((uintptr_t)d_logits & 3u) || ((uintptr_t)d_out & 3u) || ((uintptr_t)d_part & 15u))
        return fail(ctx, NIS_EALIGN, "logits and out must be 4-byte, part 16-byte aligned");
    if (!(temperature > 0.0f)) return fail(ctx, NIS_EINVAL, "temperature must be positive");
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");
    const float c = (float)(1.4426950408889634 / fmax((double)temperature, 1e-6));
    hipLaunchKernelGGL(nis::split_floor_part_kernel, dim3((unsigned)S, (unsigned)B), dim3(nis::kFPB), 0,
                       ctx->stream, d_logits, ld, (int)V, c, (int)S, (float4*)d_part);
    hipLaunchKernelGGL(nis::split_floor_merge_kernel, dim3((unsigned)B), dim3(64), 0, ctx->stream,
                       (const float4*)d_part, (int)S, c, d_out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "split stream floor launch");
}

int nis_sync(nis_ctx* ctx) {
    if (!ctx) return NIS_EINVAL;
    DeviceGuard g(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? NIS_OK : hip_fail(ctx, e, "hipStreamSynchronize");
}

}  // extern "C"

namespace {

struct OneRowStaging {
    uint64_t* state;
    uint32_t* token;
    int64_t* goff;
    uint32_t* gen;
    float* logits;
};

int check_one_args(nis_ctx* ctx, const float* h_logits, int64_t V, const nis_params* params,
                   const uint32_t* h_generated, int64_t n_generated, const uint64_t* state_inout,
                   const uint32_t* token_out) {
    if (!ctx) return NIS_EINVAL;
    if (!h_logits || !params || !state_inout || !token_out || (n_generated > 0 && !h_generated))
        return fail(ctx, NIS_EINVAL, "null pointer argument");
    if (V <= 0 || n_generated < 0) return fail(ctx, NIS_EINVAL, "bad size");
    if (V > NIS_MAX_V) return fail(ctx, NIS_ERANGE, "V exceeds NIS_MAX_V");
    if (params->reserved != 0) return fail(ctx, NIS_EINVAL, "nis_params.reserved must be 0");
    return NIS_OK;
}

// Copy one host row (and its history when the penalty applies) into the
// staging buffers, sample it on the context stream, copy the token and the
// advanced RNG state back, and wait.
int sample_one_staged(nis_ctx* ctx, const OneRowStaging& d, const float* h_logits, int64_t V,
                      const nis_params* params, const uint32_t* h_generated, int64_t n_generated,
                      bool use_gen, uint64_t state_inout[4], uint32_t* token_out) {
    hipStream_t s = ctx->stream;
    hipError_t e;
#define NIS_TRY(call, what)                           \
    do {                                              \
        e = (call);                                   \
        if (e != hipSuccess) return hip_fail(ctx, e, what); \
    } while (0)
    NIS_TRY(hipMemcpyAsync(d.logits, h_logits, (size_t)V * 4, hipMemcpyHostToDevice, s), "H2D logits");
    NIS_TRY(hipMemcpyAsync(d.state, state_inout, 32, hipMemcpyHostToDevice, s), "H2D rng");
    if (use_gen) {
        const int64_t offs[2] = {0, n_generated};
        NIS_TRY(hipMemcpyAsync(d.gen, h_generated, (size_t)n_generated * 4, hipMemcpyHostToDevice, s),
                "H2D generated");
        NIS_TRY(hipMemcpyAsync(d.goff, offs, 16, hipMemcpyHostToDevice, s), "H2D offsets");
        NIS_TRY(hipStreamSynchronize(s), "sync staging");  // `offs` is stack memory
    }
    int rc = nis_sample_batch(ctx, d.logits, V, 1, V, params, d.state, use_gen ? d.gen : nullptr,
                              use_gen ? d.goff : nullptr, d.token, nullptr);
    if (rc != NIS_OK) return rc;
    NIS_TRY(hipMemcpyAsync(token_out, d.token, 4, hipMemcpyDeviceToHost, s), "D2H token");
    NIS_TRY(hipMemcpyAsync(state_inout, d.state, 32, hipMemcpyDeviceToHost, s), "D2H rng");
    NIS_TRY(hipStreamSynchronize(s), "sync");
#undef NIS_TRY
    return NIS_OK;
}

}  // namespace

extern "C" {

int nis_sample_one(nis_ctx* ctx, const float* h_logits, int64_t V, const nis_params* params,
                   const uint32_t* h_generated, int64_t n_generated, uint64_t state_inout[4],
                   uint32_t* token_out) {
    int rc = check_one_args(ctx, h_logits, V, params, h_generated, n_generated, state_inout,
                            token_out);
    if (rc != NIS_OK) return rc;
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");

    const bool use_gen = params->repetition_penalty != 1.0f && n_generated > 0;
    auto align = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const size_t off_state = 0;
    const size_t off_tok = align(off_state + 32);
    const size_t off_goff = align(off_tok + 4);
    const size_t off_gen = align(off_goff + 16);
    const size_t off_logits = align(off_gen + (use_gen ? (size_t)n_generated * 4 : 0));
    const size_t need = align(off_logits + (size_t)V * 4);
    if (need > ctx->ws_bytes) {
        if (ctx->ws) (void)hipFree(ctx->ws);
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
        hipError_t e = hipMalloc(&ctx->ws, need);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc workspace");
        ctx->ws_bytes = need;
    }
    char* ws = (char*)ctx->ws;
    OneRowStaging d{(uint64_t*)(ws + off_state), (uint32_t*)(ws + off_tok),
                    (int64_t*)(ws + off_goff), (uint32_t*)(ws + off_gen),
                    (float*)(ws + off_logits)};
    return sample_one_staged(ctx, d, h_logits, V, params, h_generated, n_generated, use_gen,
                             state_inout, token_out);
}

int nis_sample_one_noalloc(nis_ctx* ctx, const float* h_logits, int64_t V,
                           const nis_params* params, const uint32_t* h_generated,
                           int64_t n_generated, uint64_t state_inout[4], uint32_t* token_out) {
    int rc = check_one_args(ctx, h_logits, V, params, h_generated, n_generated, state_inout,
                            token_out);
    if (rc != NIS_OK) return rc;
    if (V > NIS_NOALLOC_MAX_V)
        return fail(ctx, NIS_ERANGE, "V exceeds NIS_NOALLOC_MAX_V (the static staging area)");
    const bool use_gen = params->repetition_penalty != 1.0f && n_generated > 0;
    if (use_gen && n_generated > NIS_NOALLOC_MAX_GEN)
        return fail(ctx, NIS_ERANGE, "n_generated exceeds NIS_NOALLOC_MAX_GEN");
    DeviceGuard g(ctx->device);
    if (g.status != hipSuccess) return hip_fail(ctx, g.status, "hipSetDevice");
    void* base = nullptr;
    hipError_t e = scratch_on_device(ctx->device, &base);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
    char* ws = (char*)base;
    OneRowStaging d{(uint64_t*)(ws + kNoAllocStateOff), (uint32_t*)(ws + kNoAllocTokOff),
                    (int64_t*)(ws + kNoAllocGoffOff), (uint32_t*)(ws + kNoAllocGenOff),
                    (float*)(ws + kNoAllocLogitsOff)};
    return sample_one_staged(ctx, d, h_logits, V, params, h_generated, n_generated, use_gen,
                             state_inout, token_out);
}

#ifdef NIS_RES_TIMING
// Profiling builds only: copy the resident path's phase timestamps to the host.
int nis_debug_res_ts(void* dst, size_t bytes) {
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(nis::nis_res_ts), bytes, 0,
                                    hipMemcpyDeviceToHost);
}
#endif

#ifdef NIS_DENSE_TIMING
// Profiling builds only: copy the dense path's phase timestamps to the host.
int nis_debug_dense_ts(void* dst, size_t bytes) {
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(nis::nis_dense_ts), bytes, 0,
                                    hipMemcpyDeviceToHost);
}
#endif

#ifdef NIS_PHASE_TIMING
// Profiling builds only: copy the sparse path's phase timestamps to the host.
int nis_debug_sparse_ts(void* dst, size_t bytes) {
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(nis::nis_sparse_ts), bytes, 0,
                                    hipMemcpyDeviceToHost);
}
#endif

}  // extern "C"
