// device_common.h — order-preserving keys and wave64 / workgroup reductions
// shared by the gfx950 sampler kernels.  One workgroup = 512 lanes = 8
// wave64s (two per SIMD, so each wave may hold up to 256 VGPRs).  Every
// helper that touches LDS scratch is called by the whole workgroup (it
// contains barriers).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nis {

constexpr int kBlock = 512;
constexpr int kWaves = kBlock / 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// ---------------------------------------------------------------------------
// Order-preserving unsigned keys.  -0.0 is folded onto +0.0 first so that
// values the reference compares as equal (partial_cmp == Equal) get equal
// keys.  NaN never reaches a key (NaN rows take the special-case branch).
__device__ __forceinline__ uint32_t key32(float v) {
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float unkey32(uint32_t k) {
    const uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(b);
}
__device__ __forceinline__ uint64_t key64(double v) {
    uint64_t b = (uint64_t)__double_as_longlong(v);
    if (b == 0x8000000000000000ull) b = 0ull;
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
__device__ __forceinline__ double unkey64(uint64_t k) {
    const uint64_t b = (k >> 63) ? (k & 0x7FFFFFFFFFFFFFFFull) : ~k;
    return __longlong_as_double((long long)b);
}

// ---------------------------------------------------------------------------
// wave64 reductions (xor butterflies; the compiler lowers them to DPP /
// ds_swizzle).
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        T y = __shfl_xor(v, o);
        v = y > v ? y : v;
    }
    return v;
}
template <typename T>
__device__ __forceinline__ T wave_min(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        T y = __shfl_xor(v, o);
        v = y < v ? y : v;
    }
    return v;
}
__device__ __forceinline__ uint64_t wave_or(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o);
    return v;
}

// ---------------------------------------------------------------------------
// DPP wave64 scans and reductions (all 64 lanes must be active).  Inclusive
// Hillis-Steele scan inside each 16-lane row (row_shr:1,2,4,8), then
// row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3.  These
// stay in the VALU (no LDS round trip, unlike __shfl_*).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp0(uint32_t v) {  // out-of-row lanes read 0
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, true);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_ninf(float v) {  // out-of-row lanes read -inf
    return __int_as_float(__builtin_amdgcn_update_dpp((int)0xFF800000u, __float_as_int(v), CTRL,
                                                      ROW_MASK, 0xF, false));
}
__device__ __forceinline__ uint32_t wscan_u32(uint32_t v) {
    v += dpp0<0x111>(v);
    v += dpp0<0x112>(v);
    v += dpp0<0x114>(v);
    v += dpp0<0x118>(v);
    v += dpp0<0x142, 0xA>(v);
    v += dpp0<0x143, 0xC>(v);
    return v;
}
__device__ __forceinline__ float wscan_f32(float v) {
#define NIS_DPPF(C, M) __uint_as_float(dpp0<C, M>(__float_as_uint(v)))
    v += NIS_DPPF(0x111, 0xF);
    v += NIS_DPPF(0x112, 0xF);
    v += NIS_DPPF(0x114, 0xF);
    v += NIS_DPPF(0x118, 0xF);
    v += NIS_DPPF(0x142, 0xA);
    v += NIS_DPPF(0x143, 0xC);
#undef NIS_DPPF
    return v;
}
__device__ __forceinline__ double wscan_f64(double v) {
#define NIS_DPPD(C, M)                                                        \
    {                                                                          \
        const uint64_t b = (uint64_t)__double_as_longlong(v);                  \
        const uint64_t lo = dpp0<C, M>((uint32_t)b), hi = dpp0<C, M>((uint32_t)(b >> 32)); \
        v += __longlong_as_double((long long)((hi << 32) | lo));              \
    }
    NIS_DPPD(0x111, 0xF)
    NIS_DPPD(0x112, 0xF)
    NIS_DPPD(0x114, 0xF)
    NIS_DPPD(0x118, 0xF)
    NIS_DPPD(0x142, 0xA)
    NIS_DPPD(0x143, 0xC)
#undef NIS_DPPD
    return v;
}
__device__ __forceinline__ float wscan_max_f32(float v) {
    v = fmaxf(v, dpp_ninf<0x111>(v));
    v = fmaxf(v, dpp_ninf<0x112>(v));
    v = fmaxf(v, dpp_ninf<0x114>(v));
    v = fmaxf(v, dpp_ninf<0x118>(v));
    v = fmaxf(v, dpp_ninf<0x142, 0xA>(v));
    v = fmaxf(v, dpp_ninf<0x143, 0xC>(v));
    return v;
}
// Wave totals, uniform across the wave (lane 63 holds the inclusive total).
__device__ __forceinline__ uint32_t wsum_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readlane((int)wscan_u32(v), 63);
}
__device__ __forceinline__ float wsum_f32(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wscan_f32(v)), 63));
}
__device__ __forceinline__ double wsum_f64(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(wscan_f64(v));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ float wmax_f32(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wscan_max_f32(v)), 63));
}
// Number of set bits of `mask` below this lane (the lane's slot in a
// wave-compacted append).
__device__ __forceinline__ uint32_t lane_rank(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
// Wave-uniform broadcast of lane `src` (src itself wave-uniform).
__device__ __forceinline__ uint32_t bcast_u32(uint32_t v, int src) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, src);
}
__device__ __forceinline__ float bcast_f32(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ __forceinline__ double bcast_f64(double v, int src) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, src);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), src);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Workgroup reductions.  `scr` is LDS scratch of at least kWaves elements;
// the leading barrier makes back-to-back calls on the same scratch safe.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scr) {
    v = wave_sum(v);
    __syncthreads();
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    T r = scr[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) r += scr[i];
    return r;
}
template <typename T>
__device__ __forceinline__ T block_max(T v, T* scr) {
    v = wave_max(v);
    __syncthreads();
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    T r = scr[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) r = scr[i] > r ? scr[i] : r;
    return r;
}
template <typename T>
__device__ __forceinline__ T block_min(T v, T* scr) {
    v = wave_min(v);
    __syncthreads();
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    T r = scr[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) r = scr[i] < r ? scr[i] : r;
    return r;
}
__device__ __forceinline__ uint64_t block_or(uint64_t v, uint64_t* scr) {
    v = wave_or(v);
    __syncthreads();
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    uint64_t r = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) r |= scr[i];
    return r;
}

// Inclusive workgroup scan in lane order (thread 0 first).  Returns the
// inclusive prefix of this thread; *total receives the workgroup total,
// which equals the last thread's inclusive prefix bit for bit.
template <typename T>
__device__ __forceinline__ T block_inclusive_scan(T v, T* scr, T* total) {
    const int l = lane_id(), w = wave_id();
    T incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        T y = __shfl_up(incl, o);
        if (l >= o) incl += y;
    }
    __syncthreads();
    if (l == 63) scr[w] = incl;
    __syncthreads();
    T base = T(0);
    T tot = T(0);
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        if (i < w) base += scr[i];
        if (i < kWaves - 1) tot += scr[i];
    }
    // `base` of the last wave and `tot` add scr[0 .. kWaves-2] in the same
    // order, so the last thread's inclusive prefix equals the total.
    tot += scr[kWaves - 1];
    *total = tot;
    return (w == 0) ? incl : base + incl;
}

}  // namespace nis
