// device_common.h — order-preserving keys and wave64 / workgroup reductions
// shared by the gfx950 sampler kernels.  One workgroup = 1024 lanes = 16
// wave64s; every helper that touches LDS scratch is called by the whole
// workgroup (it contains barriers).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nis {

constexpr int kBlock = 1024;
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
    // Both `base` for the last wave and `tot` sum scr[0..14] in the same
    // order, so the last thread's inclusive prefix equals the total.
    tot += scr[kWaves - 1];
    *total = (w == kWaves - 1) ? tot : tot;
    return (w == 0) ? incl : base + incl;
}

}  // namespace nis
