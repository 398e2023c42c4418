// penalty_bits.h — a row's repetition-penalty history as LDS bitmaps, for the
// 1024-lane register-resident kernels (apply_repetition_penalty,
// src/sampler.rs:83-101).
//
// The row's float4 slots are laid out as in those kernels: chunk k / lane l of
// a wave holds slot wbase + 64 k + l, element q of slot s being row index
// 4 s + q - mis.  The history's ids set, per slot, a bit (pslot) and a 4-bit
// mask of its penalised elements (pnib).  Each wave then keeps one bit per
// chunk (pany: some slot of the chunk holds a penalised element) and each
// lane the masks of its own slots (pnl, 4 bits per chunk), so a chunk costs
// one scalar test unless it holds a penalised element.
//
// Protocol (every lane of the workgroup takes part):
//   pen_load_ids   after the first chunk's load is issued (global loads);
//   pen_clear      before the workgroup's first barrier;
//   pen_set_bits   after it, then a second barrier;
//   pen_masks      after that one.
#pragma once
#include "general_path.h"

namespace nis {

constexpr int kPB = 1024;                    // lanes of the workgroups using this
constexpr int kPMaxV = 53245;                // their largest row
constexpr int kPHist = 4 * kPB;              // history entries per row (raw, with repeats)
constexpr int kPNibW = kPMaxV / 32 + 2;      // words of 4-bit slot masks (8 slots per word)
constexpr int kPSlW = kPMaxV / 256 + 2;      // slot bitmap words (64-bit)

struct PenBits {
    unsigned long long pslot[kPSlW];  // bit s: float4 slot s holds a penalised element
    uint32_t pnib[kPNibW];            // bits 4 (s % 8) + q of word s / 8: element q of slot s
};

// The row's raw history ids, kPHist / kPB per lane (0xFFFFFFFF: none).
// Returns true when the history is longer than kPHist (the row is declined).
__device__ __forceinline__ bool pen_load_ids(const RowArgs& a, int row, int tid,
                                             uint32_t (&hid)[kPHist / kPB]) {
    if (a.gen_len != nullptr) {
        // a decode step: the history's slots are known before its length, so
        // both loads go out at once and the length masks the ids after
        const int64_t g0 = (int64_t)row * a.gen_cap;
        const int nc = (int)min(a.gen_cap, (int64_t)kPHist);
#pragma unroll
        for (int i = 0; i < kPHist / kPB; ++i) {
            const int j = tid + kPB * i;
            hid[i] = (j < nc) ? a.gen_ids[g0 + j] : 0xFFFFFFFFu;
        }
        const int nh = (int)min((int64_t)max(a.gen_len[row], 0), a.gen_cap);
#pragma unroll
        for (int i = 0; i < kPHist / kPB; ++i)
            if (tid + kPB * i >= nh) hid[i] = 0xFFFFFFFFu;
        return nh > kPHist;
    }
    int64_t g0 = 0, g1 = 0;
    if (!gen_range(a, row, g0, g1)) g1 = g0;
    const int nh = (int)min(g1 - g0, (int64_t)kPHist);
#pragma unroll
    for (int i = 0; i < kPHist / kPB; ++i) {
        const int j = tid + kPB * i;
        hid[i] = (j < nh) ? a.gen_ids[g0 + j] : 0xFFFFFFFFu;
    }
    return g1 - g0 > (int64_t)kPHist;
}

__device__ __forceinline__ void pen_clear(PenBits& pb, int tid) {
    pb.pnib[tid] = 0u;
    if (tid + kPB < kPNibW) pb.pnib[tid + kPB] = 0u;
    if (tid < kPSlW) pb.pslot[tid] = 0ull;
}

__device__ __forceinline__ void pen_set_bits(PenBits& pb, const uint32_t (&hid)[kPHist / kPB], int V,
                                             int mis) {
#pragma unroll
    for (int i = 0; i < kPHist / kPB; ++i) {
        const uint32_t id = hid[i];
        if (id < (uint32_t)V) {
            const uint32_t f = id + (uint32_t)mis;  // float position from the slot base
            atomicOr(&pb.pnib[f >> 5], 1u << (f & 31u));
            atomicOr(reinterpret_cast<uint32_t*>(&pb.pslot[0]) + (f >> 7), 1u << ((f >> 2) & 31u));
        }
    }
}

// pany (wave-uniform) and pnl (this lane) for a wave owning slots
// [wbase, wbase + 64 Kw), wbase a multiple of 64, at most NCH chunks.
template <int NCH>
__device__ __forceinline__ void pen_masks(const PenBits& pb, int wbase, int Kw, int l,
                                          uint32_t& pany, uint64_t& pnl) {
    const unsigned long long m = (l < Kw) ? pb.pslot[(wbase >> 6) + min(l, NCH - 1)] : 0ull;
    pany = (uint32_t)__ballot(m != 0ull);
    pnl = 0ull;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        if ((pany >> k) & 1u) {
            const uint32_t s = (uint32_t)(wbase + l + 64 * k);
            pnl |= (uint64_t)((pb.pnib[s >> 3] >> (4u * (s & 7u))) & 15u) << (4 * k);
        }
    }
}

// apply_repetition_penalty's update of one logit (sampler.rs:94-98), in f64.
__device__ __forceinline__ double pen_value(float x, double pen) {
    return (x > 0.0f) ? (double)x / pen : (double)x * pen;
}

// 2^(yc - R) in f64 for a penalised value (yc = y c in f64): the f32 exp2 of
// the fractional part, scaled exactly.
__device__ __forceinline__ double pen_mass(double yc, float R) {
    const double d = yc - (double)R;
    if (!(d == d)) return d;  // NaN stays NaN (the row is declined through Z)
    if (d < -1100.0) return 0.0;
    if (d > 1100.0) return INFINITY;
    const double fl = floor(d);
    return ldexp((double)__builtin_amdgcn_exp2f((float)(d - fl)), (int)fl);
}

// The smallest float >= y (y finite or infinite; NaN passes through).
__device__ __forceinline__ float pen_f32_up(double y) {
    const float f = (float)y;
    if (!((double)f < y)) return f;
    if (f == 0.0f) return __uint_as_float(1u);  // the least positive float
    const uint32_t b = __float_as_uint(f);
    return __uint_as_float(f > 0.0f ? b + 1u : b - 1u);  // (FLT_MAX + 1 ulp: +inf)
}

}  // namespace nis
