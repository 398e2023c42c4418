// kernels.h — __global__ entry points of the sampler library (gfx950).
#pragma once
#include "sparse_path.h"
#include "resident_path.h"
#include "dense_path.h"
#include "long_path.h"
#include "long_sparse_path.h"

namespace nis {

// One 512-lane workgroup per row on the general path: the launches no
// row kernel takes (V < 256, top-p <= 0, top-k with a penalty history or on
// rows longer than the registers hold, a penalty history on rows longer
// than the registers hold).
__global__ __launch_bounds__(kBlock) void sample_rows_kernel(RowArgs a) {
    __shared__ GeneralShared sh;
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;  // a finished sequence (decode step)
    general_row(a, row, sh, NIS_REJECT_SHAPE);
}

// Sparse top-p rows: one 1024-lane workgroup per row.  A row the sparse
// path declines (or cannot take) runs the general path on the first 512
// lanes; the other waves leave first, so the general path's barriers count
// only its own eight waves.  PEN: the launch carries a repetition-penalty
// history, applied inside the sparse path.  TOPK: the launch carries a top-k
// (sampler.rs:103-116), applied inside the sparse path.
template <bool PEN, bool TOPK = false>
__device__ __forceinline__ void sparse_rows_body(const RowArgs& a) {
    __shared__ union {
        GeneralShared g;
        WideShared s;
    } sh;
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;  // a finished sequence (decode step)
    asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.temperature), "s"(a.top_p),
                 "s"(a.penalty), "s"(a.top_k), "s"(a.gen_ids), "s"(a.gen_off));
    uint32_t reject = NIS_REJECT_SHAPE;
    if (sparse_eligible<PEN, TOPK>(a, row)) {
        reject = sparse_row<PEN, TOPK>(a, row, sh.s);
        if (reject == NIS_REJECT_NONE) return;
    }
    if (threadIdx.x >= kBlock) return;
    __syncthreads();
    general_row<1>(a, row, sh.g, reject);
}
__global__ __launch_bounds__(kSB) void sample_rows_sparse_kernel(RowArgs a) {
    sparse_rows_body<false>(a);
}
// Sparse top-p rows with a repetition-penalty history.  A row the sparse
// path declines (most often a long history: more penalised elements in a
// wave's range than its side lists hold) gets the token kLPending | reason,
// and sample_rows_dense_pending_kernel, launched after it, finishes exactly
// those rows (the sparse path has written nothing when it declines).
__global__ __launch_bounds__(kSB) void sample_rows_sparse_pen_kernel(RowArgs a) {
    __shared__ WideShared sh;
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;  // a finished sequence (decode step)
    asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.temperature), "s"(a.top_p),
                 "s"(a.penalty), "s"(a.top_k), "s"(a.gen_ids), "s"(a.gen_off));
    uint32_t reject = NIS_REJECT_SHAPE;
    if (sparse_eligible<true, false>(a, row)) {
        reject = sparse_row<true, false>(a, row, sh);
        if (reject == NIS_REJECT_NONE) return;
    }
    if (threadIdx.x == 0) a.tokens[row] = kLPending | reject;
}

// The rows a penalised sparse launch declined (token kLPending | reason): the
// dense path, which takes any nucleus and up to 16 penalised elements per
// lane, then the general path (first 512 lanes) if that declines too.  One
// 1024-lane workgroup per row; a row not pending costs one token read.
__global__ __launch_bounds__(kDB) void sample_rows_dense_pending_kernel(RowArgs a) {
    __shared__ DenseKernelShared sh;
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;
    const uint32_t t = a.tokens[row];
    if ((t & kLPending) != kLPending) return;
    asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.temperature), "s"(a.top_p),
                 "s"(a.penalty), "s"(a.gen_ids), "s"(a.gen_off));
    __syncthreads();  // (every lane has read the marker before any result overwrites it)
    uint32_t reject = t & ~kLPending;
    if (dense_eligible<true>(a, row)) {
        reject = dense_row<true>(a, row, sh.d);
        if (reject == NIS_REJECT_NONE) return;
    }
    if (threadIdx.x >= kBlock) return;
    __syncthreads();
    general_row<1>(a, row, sh.g, reject);
}
__global__ __launch_bounds__(kSB) void sample_rows_sparse_topk_kernel(RowArgs a) {
    sparse_rows_body<false, true>(a);
}

// Top-p rows longer than the registers hold, read once: one 1024-lane
// workgroup per row.  A row the single-read path declines runs the long-row
// method (which reads it again) on the first 512 lanes, and the general path
// when that declines too; the other waves leave first, as above.
__global__ __launch_bounds__(kLSB) void sample_rows_long_sparse_kernel(RowArgs a) {
    __shared__ union {
        LSShared s;
        LongShared lg;
        GeneralShared g;
    } sh;
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;  // a finished sequence (decode step)
    asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.temperature), "s"(a.top_p),
                 "s"(a.penalty), "s"(a.top_k), "s"(a.gen_ids), "s"(a.gen_off));
    uint32_t reject = NIS_REJECT_SHAPE;
    if (lsparse_eligible(a, row)) {
        reject = lsparse_row(a, row, sh.s);
        if (reject == NIS_REJECT_NONE) return;
    }
    if (threadIdx.x >= kLB) return;
    __syncthreads();
    if (long_eligible<kLongTopP>(a, row)) {
        reject = long_row<kLongTopP>(a, row, sh.lg, reject);
        if (reject == NIS_REJECT_NONE) return;
        __syncthreads();
    }
    general_row<1>(a, row, sh.g, reject);
}

// General path only (used by tests to cross-check the two paths).
__global__ __launch_bounds__(kBlock) void sample_rows_general_kernel(RowArgs a) {
    __shared__ GeneralShared sh;
    general_row(a, (int)blockIdx.x, sh, NIS_REJECT_NONE);
}

// Rng::new per row (sampler.rs:46-56).
__global__ void rng_seed_kernel(const uint64_t* __restrict__ seeds, int32_t B,
                                uint64_t* __restrict__ states) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    uint64_t s[4];
    rng_seed(seeds[b], s);
    states[4 * b + 0] = s[0];
    states[4 * b + 1] = s[1];
    states[4 * b + 2] = s[2];
    states[4 * b + 3] = s[3];
}

// apply_repetition_penalty (sampler.rs:83-101) on one f64 row: the distinct
// ids are collected in an LDS bitmap, then each is penalised once.
__global__ __launch_bounds__(kBlock) void repetition_penalty_kernel(
    double* __restrict__ logits, int64_t V, const uint32_t* __restrict__ gen, int64_t n_gen,
    double penalty) {
    __shared__ uint32_t bitmap[NIS_MAX_V / 32];
    const int64_t nw = (V + 31) >> 5;
    for (int64_t i = threadIdx.x; i < nw; i += kBlock) bitmap[i] = 0u;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n_gen; i += kBlock) {
        const uint32_t id = gen[i];
        if ((int64_t)id < V) atomicOr(&bitmap[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
    for (int64_t w = threadIdx.x; w < nw; w += kBlock) {
        uint32_t bits = bitmap[w];
        while (bits) {
            const int b = __ffs(bits) - 1;
            bits &= bits - 1;
            const int64_t j = w * 32 + b;
            const double v = logits[j];
            logits[j] = (v > 0.0) ? v / penalty : v * penalty;
        }
    }
}

}  // namespace nis
