// floor_path.h — the stream floor: the sparse kernel's row layout and load
// pipeline (one 1024-lane workgroup per row, wave w owning the contiguous
// chunks [cpw w, cpw (w + 1)) of the row's float4 slots, three nontemporal
// 16-byte buffer loads in flight per lane, the later waves at a higher
// priority) with only the work every element needs in any sampler: its
// max and its mass 2^(x c - R_w) summed in f64.  After each row's last byte
// there are two wave reductions and one barrier.  It samples nothing; its
// launch time is the bandwidth floor the sparse kernel is measured against
// (nis_stream_floor, bench.py --floor).
//
// The split floor (nis_stream_floor_split, bench.py --floor --split S): the
// same work with each row split over S workgroups of 256 lanes, each wave
// writing its slice's max and mass sum at its own reference, and a second
// launch merging a row's 4 S partials.  Any sampler that splits a row over
// workgroups does at least this (one slice stream and one merge launch) for
// each of its merges, so its time bounds such a design from below.
#pragma once
#include "sparse_path.h"

namespace nis {

struct FloorShared {
    double z[kSW];
    float m[kSW];
    float r[kSW];
};

__global__ __launch_bounds__(kSB) void stream_floor_kernel(const float* __restrict__ logits,
                                                           int64_t ld, int V, float c,
                                                           float* __restrict__ out) {
    __shared__ FloorShared sh;
    const int row = (int)blockIdx.x;
    const int l = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const gfp rowp = (gfp)(logits + (int64_t)row * ld);
    const int mis = (int)(((uintptr_t)rowp >> 2) & 3);
    const gf4p base = (gf4p)(rowp - mis);
    const int f_lo = mis ? 1 : 0;
    const int f_hi = (V + mis - 4) >> 2;
    const int nsl = (V + mis + 3) >> 2;
    const int cpw = (((nsl + 63) >> 6) + kSW - 1) / kSW;
    const int wbase = 64 * cpw * w;
    const int Kw = min(max((nsl - wbase + 63) >> 6, 0), cpw);
    const int slot0 = wbase + l;
    // the (at most 3 + 3) elements of partial head / tail slots (lane i < 3:
    // element i, lane 3 + i: element V - 6 + 3 + i); the buffer descriptor
    // covers the whole slots [0, f_hi], the partial head slot is redirected
    // to f_lo and slots past f_hi read zeros (both fixed below)
    const float hv = rowp[(l < 3) ? l : ((l < 6) ? V - 6 + l : 0)];
    const uint64_t bptr = (uint64_t)(uintptr_t)base;
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    const int voff = 16 * slot0;  // (chunks past the first never hold slot 0)
    f4v xv[kSN];
#define NIS_FLOAD(k)                                                                         \
    do {                                                                                     \
        xv[k] = nis_buffer_load_f4(                                                          \
            rsrc, ((k) < Kw) ? ((k) == 0 ? 16 * max(slot0, f_lo) : voff + 1024 * (k)) : 0x7FFFFFF0, \
            0, 2);                                                                           \
    } while (0)
#pragma unroll
    for (int k = 0; k < kSD; ++k) {
        NIS_FLOAD(k);
        __builtin_amdgcn_sched_barrier(0);
    }
    const bool edge_wave = (wbase < f_lo) || (wbase + 64 * Kw - 1 > f_hi);
    const float h0 = bcast_f32(hv, 0), h1 = bcast_f32(hv, 1), h2 = bcast_f32(hv, 2);
    const float t0 = bcast_f32(hv, 3), t1 = bcast_f32(hv, 4), t2 = bcast_f32(hv, 5);
#define NIS_FFIX(k)                                                                           \
    do {                                                                                      \
        const int fb0 = wbase + (k) * 64;                                                     \
        if (edge_wave && (fb0 < f_lo || fb0 + 63 > f_hi))                                     \
            xv[k] = fix_slot(xv[k], slot0 + (k) * 64, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2); \
    } while (0)
    __builtin_amdgcn_s_setprio(0);
    if (w >= kSW / 4) __builtin_amdgcn_s_setprio(1);
    if (w >= kSW / 2) __builtin_amdgcn_s_setprio(2);
    if (w >= 3 * kSW / 4) __builtin_amdgcn_s_setprio(3);
    const f4v ninf4 = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    if (Kw == 0) xv[0] = ninf4;
    else NIS_FFIX(0);
    const float m0 = wmax_f32(max4(xv[0]));
    const float Rw = (m0 > -INFINITY && fabsf(m0 * c) < 1e30f) ? ceilf(m0 * c) : 0.0f;
    double z = 0.0;
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kSN; ++k) {
        if (k + kSD < kSN) NIS_FLOAD(k + kSD);
        __builtin_amdgcn_sched_barrier(0);
        if (k >= Kw) continue;
        if (k > 0) NIS_FFIX(k);
        const f4v x = xv[k];
        const float e0 = __builtin_amdgcn_exp2f(fmaf(x.x, c, -Rw));
        const float e1 = __builtin_amdgcn_exp2f(fmaf(x.y, c, -Rw));
        const float e2 = __builtin_amdgcn_exp2f(fmaf(x.z, c, -Rw));
        const float e3 = __builtin_amdgcn_exp2f(fmaf(x.w, c, -Rw));
        z += (double)((e0 + e1) + (e2 + e3));
        mx = fmaxf(mx, max4(x));
    }
#undef NIS_FLOAD
#undef NIS_FFIX
    __builtin_amdgcn_s_setprio(0);
    mx = wmax_f32(mx);
    z = wsum_f64(z);
    if (l == 0) {
        sh.z[w] = z;
        sh.m[w] = mx;
        sh.r[w] = Rw;
    }
    lds_barrier();
    if (w == 0) {
        const bool rv = l < kSW;
        const float M = wmax_f32(rv ? sh.m[l] : -INFINITY);
        const float R = (M > -INFINITY && fabsf(M * c) < 1e30f) ? ceilf(M * c) : 0.0f;
        const double Z = wsum_f64(rv && sh.m[l] > -INFINITY ? ldexp(sh.z[l], (int)(sh.r[l] - R)) : 0.0);
        if (l == 0) {
            out[2 * (int64_t)row] = M;
            out[2 * (int64_t)row + 1] = (float)Z;  // sum of 2^(x c - ceil(M c))
        }
    }
}

constexpr int kFPB = 256;  // lanes per workgroup of the split floor
constexpr int kFPN = 16;   // float4 slots per lane (at most): a slice of 4096 slots

// Wave (s, w) of row b: slots lo + 256 i + tid of the row's float4 slots,
// lo = s Q, Q = ceil(nsl / S); part[(b S + s) 4 + w] = {z (f64 bits), max, R}.
__global__ __launch_bounds__(kFPB) void split_floor_part_kernel(const float* __restrict__ logits,
                                                               int64_t ld, int V, float c, int S,
                                                               float4* __restrict__ part) {
    const int row = (int)blockIdx.y, s = (int)blockIdx.x;
    const int l = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int tid = (int)threadIdx.x;
    const gfp rowp = (gfp)(logits + (int64_t)row * ld);
    const int mis = (int)(((uintptr_t)rowp >> 2) & 3);
    const int f_lo = mis ? 1 : 0;
    const int f_hi = (V + mis - 4) >> 2;
    const int nsl = (V + mis + 3) >> 2;
    const int Q = (nsl + S - 1) / S;
    const int lo = s * Q, hi = min(nsl, lo + Q);
    const float hv = rowp[(l < 3) ? l : ((l < 6) ? V - 6 + l : 0)];
    const uint64_t bptr = (uint64_t)(uintptr_t)(rowp - mis);
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    f4v xv[kFPN];
#pragma unroll
    for (int i = 0; i < kFPN; ++i) {
        const int f = lo + tid + kFPB * i;
        xv[i] = nis_buffer_load_f4(rsrc, f < hi ? 16 * max(f, f_lo) : 0x7FFFFFF0, 0, 2);
    }
    const float h0 = bcast_f32(hv, 0), h1 = bcast_f32(hv, 1), h2 = bcast_f32(hv, 2);
    const float t0 = bcast_f32(hv, 3), t1 = bcast_f32(hv, 4), t2 = bcast_f32(hv, 5);
    const f4v ninf4 = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kFPN; ++i) {
        const int f = lo + tid + kFPB * i;
        xv[i] = f < hi ? fix_slot(xv[i], f, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2) : ninf4;
        mx = fmaxf(mx, max4(xv[i]));
    }
    mx = wmax_f32(mx);
    const float R = (mx > -INFINITY && fabsf(mx * c) < 1e30f) ? ceilf(mx * c) : 0.0f;
    double z = 0.0;
#pragma unroll
    for (int i = 0; i < kFPN; ++i) {
        const f4v x = xv[i];
        z += (double)((__builtin_amdgcn_exp2f(fmaf(x.x, c, -R)) + __builtin_amdgcn_exp2f(fmaf(x.y, c, -R))) +
                      (__builtin_amdgcn_exp2f(fmaf(x.z, c, -R)) + __builtin_amdgcn_exp2f(fmaf(x.w, c, -R))));
    }
    z = wsum_f64(z);
    if (l == 0) {
        const uint64_t zb = (uint64_t)__double_as_longlong(z);
        part[((int64_t)row * S + s) * 4 + w] =
            float4{__uint_as_float((uint32_t)zb), __uint_as_float((uint32_t)(zb >> 32)), mx, R};
    }
}

// One wave per row: the row's 4 S partials merged (max, then the sums at
// R = ceil(max c)), as stream_floor_kernel writes them.
__global__ __launch_bounds__(64) void split_floor_merge_kernel(const float4* __restrict__ part, int S,
                                                               float c, float* __restrict__ out) {
    const int row = (int)blockIdx.x;
    const int l = (int)threadIdx.x;
    const int n = 4 * S;
    float m = -INFINITY;
    for (int i = l; i < n; i += 64) m = fmaxf(m, part[(int64_t)row * n + i].z);
    const float M = wmax_f32(m);
    const float R = (M > -INFINITY && fabsf(M * c) < 1e30f) ? ceilf(M * c) : 0.0f;
    double z = 0.0;
    for (int i = l; i < n; i += 64) {
        const float4 p = part[(int64_t)row * n + i];
        const double zi = __longlong_as_double((long long)(((uint64_t)__float_as_uint(p.y) << 32) |
                                                           __float_as_uint(p.x)));
        z += p.z > -INFINITY ? ldexp(zi, (int)(p.w - R)) : 0.0;
    }
    const double Z = wsum_f64(z);
    if (l == 0) {
        out[2 * (int64_t)row] = M;
        out[2 * (int64_t)row + 1] = (float)Z;
    }
}

}  // namespace nis
