// floor_path.h — the stream floor: the sparse kernel's row layout and load
// pipeline (one 1024-lane workgroup per row, wave w owning the contiguous
// chunks [cpw w, cpw (w + 1)) of the row's float4 slots, three nontemporal
// 16-byte buffer loads in flight per lane, the later waves at a higher
// priority) with only the work every element needs in any sampler: its
// max and its mass 2^(x c - R_w) summed in f64.  After each row's last byte
// there are two wave reductions and one barrier.  It samples nothing; its
// launch time is the bandwidth floor the sparse kernel is measured against
// (nis_stream_floor, bench.py --floor).
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

}  // namespace nis
