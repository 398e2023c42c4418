// resident_path.h — one row per 1024-lane workgroup (16 wave64s, four per
// SIMD), the row held in VGPRs (V <= 53245): nis_sample_batch for greedy
// rows and top-p off (src/sampler.rs:163-217).
//
// Layout.  The row's float4 slots are split over the 16 waves in whole
// 64-slot chunks, cpw per wave: chunk k / lane l of wave w holds slot
// 64 (cpw w + k) + l, so each wave owns a contiguous index range and inside
// it index order is chunk, lane, element.  Every lane keeps kRD loads in
// flight ahead of the chunk it works on, so every wave's data arrives over
// the whole stream.
//
// Masses.  2^(x c - R) with c = log2(e) / T split as c_hi + c_lo (both f32,
// c_hi = f32(c)): the product of x with c's rounding error is recovered by a
// second fma, so a mass depends on the depth below the maximum only through
// the last rounding of its argument.  In the stream, R is an integer
// reference of the wave that follows its running max, and the masses are
// f32, summed in f64.  The helpers for exact fixed-point masses of one
// element (r_fm: 2^f * 2^24 rounded down, f = fma(x, c_lo, fma(x, c_hi, -o))
// the fraction above octave o; r_key: the stable order as one key) serve the
// dense and long-row kernels.
//
// Top-p off: every element is kept; the walk goes waves -> chunks -> lanes
// -> elements over the stream's own f32 masses (chunk totals from one
// transposed LDS sum in the chosen wave), and the drawn token's probability
// uses its exact mass.
// Greedy (sampler.rs:172-181): the first index of the maximum.
//
// Any row this path cannot prove (non-finite values, a reference range too
// wide for f32 masses) returns a reject code before anything is written, and
// the caller runs the general path on it.
#pragma once
#include "row_common.h"
#include "penalty_bits.h"

namespace nis {

constexpr int kRB = 1024;                  // lanes per workgroup
constexpr int kRW = kRB / 64;              // waves per workgroup
constexpr int kRN = 13;                    // float4 chunks per lane (at most)
constexpr int kRMaxV = kRB * 4 * kRN - 3;  // 53245
constexpr int kRD = 3;                     // loads in flight per lane ahead of the one in use
enum { kResAll = 1, kResGreedy = 2, kResGreedyPen = 3, kResAllPen = 4 };
static_assert(kRB == kPB && kRMaxV == kPMaxV, "penalty bitmaps sized for this layout");

// Optional phase timestamps (profiling builds only, compiled out unless
// NIS_RES_TIMING is defined): each wave keeps the 100 MHz clock of its phases
// in registers and lane 0 stores them when the wave is done, at slot
// 8 * (16 * row + wave) + i (a store per phase would perturb the phases).
#ifdef NIS_RES_TIMING
__device__ unsigned long long nis_res_ts[2048 * kRW * 16];
#define NIS_RTDECL unsigned long long nis_t_[16] = {};
#define NIS_RTS(i) (nis_t_[i] = wall_clock64())
#define NIS_RTFLUSH()                                                                  \
    do {                                                                               \
        if (lane_id() == 0 && blockIdx.x < 2048) {                                     \
            _Pragma("unroll") for (int i_ = 0; i_ < 16; ++i_)                           \
                nis_res_ts[16 * (kRW * blockIdx.x + wave_id()) + i_] = nis_t_[i_];      \
        }                                                                              \
    } while (0)
#else
#define NIS_RTDECL
#define NIS_RTS(i) \
    do {           \
    } while (0)
#define NIS_RTFLUSH() \
    do {              \
    } while (0)
#endif

// A member of a cutoff bucket (dense and long-row kernels): its logit, row
// index, octave and octave-relative fixed-point mass.
struct alignas(16) RCand {
    float x;
    uint32_t idx;
    int32_t b;
    uint32_t fm;
};
// Stream-end record of one wave (lane 0 writes it).
struct alignas(16) RRec {
    double z;      // sum of 2^(x c - R_w) over the wave's elements (greedy with a
                   // penalty: the wave's largest penalised value, f64)
    float mx;      // wave max logit
    float rw;      // R_w
    float thc;     // greedy: the first index of the wave max
    uint32_t nc;   // top-p off with stats: the wave's elements above -inf (greedy
                   // with a penalty: the first index of that penalised value)
    uint32_t bad;  // the wave saw input this path does not take
    uint32_t pad;
};

struct ResShared {
    float s4[kRW][kRN][64];  // top-p off: per-chunk per-lane f32 masses
    RRec rec[kRW];
    double u0;               // the draw
    PenBits pb;              // with a penalty: the history's bitmaps
    float pmx[kRW];          // top-p off with a penalty: each wave's penalised max, rounded up
    double pymx[kRW];        //   and exact (f64)
};

// u64 wave sum: DPP row sums, then the four row totals (uniform).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned long long rdpp_u64(unsigned long long v);
__device__ __forceinline__ unsigned long long rbcast_u64(unsigned long long v, int src);
__device__ __forceinline__ unsigned long long wsum_u64(unsigned long long v) {
    v += rdpp_u64<0x111, 0xF>(v);
    v += rdpp_u64<0x112, 0xF>(v);
    v += rdpp_u64<0x114, 0xF>(v);
    v += rdpp_u64<0x118, 0xF>(v);
    return (rbcast_u64(v, 15) + rbcast_u64(v, 31)) + (rbcast_u64(v, 47) + rbcast_u64(v, 63));
}

// u64 inclusive wave scan and broadcast (lo / hi words moved by DPP).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned long long rdpp_u64(unsigned long long v) {
    const uint32_t lo = dpp0<CTRL, ROW_MASK>((uint32_t)v), hi = dpp0<CTRL, ROW_MASK>((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long rscan_u64w(unsigned long long v) {
    v += rdpp_u64<0x111, 0xF>(v);
    v += rdpp_u64<0x112, 0xF>(v);
    v += rdpp_u64<0x114, 0xF>(v);
    v += rdpp_u64<0x118, 0xF>(v);
    v += rdpp_u64<0x142, 0xA>(v);
    v += rdpp_u64<0x143, 0xC>(v);
    return v;
}
__device__ __forceinline__ unsigned long long rbcast_u64(unsigned long long v, int src) {
    return ((unsigned long long)bcast_u32((uint32_t)(v >> 32), src) << 32) | bcast_u32((uint32_t)v, src);
}
// f64 inclusive scan over lanes 0..15 (one DPP row).
__device__ __forceinline__ double rscan16_f64(double v) {
#define NIS_RD16(C)                                                                    \
    {                                                                                  \
        const uint64_t b_ = (uint64_t)__double_as_longlong(v);                         \
        const uint64_t lo_ = dpp0<C, 0xF>((uint32_t)b_), hi_ = dpp0<C, 0xF>((uint32_t)(b_ >> 32)); \
        v += __longlong_as_double((long long)((hi_ << 32) | lo_));                     \
    }
    NIS_RD16(0x111)
    NIS_RD16(0x112)
    NIS_RD16(0x114)
    NIS_RD16(0x118)
#undef NIS_RD16
    return v;
}
__device__ __forceinline__ unsigned long long rscan16_u64(unsigned long long v) {
    v += rdpp_u64<0x111, 0xF>(v);
    v += rdpp_u64<0x112, 0xF>(v);
    v += rdpp_u64<0x114, 0xF>(v);
    v += rdpp_u64<0x118, 0xF>(v);
    return v;
}

// DPP u32 min over the wave (out-of-row lanes read the identity), uniform.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_umin_id(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)0xFFFFFFFFu, (int)v, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ uint32_t wmin_u32(uint32_t v) {
    v = min(v, dpp_umin_id<0x111>(v));
    v = min(v, dpp_umin_id<0x112>(v));
    v = min(v, dpp_umin_id<0x114>(v));
    v = min(v, dpp_umin_id<0x118>(v));
    v = min(v, dpp_umin_id<0x142, 0xA>(v));
    v = min(v, dpp_umin_id<0x143, 0xC>(v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// max of a float4 without the canonicalising moves of fmaxf
__device__ __forceinline__ float r_max4(const f4v& v) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(v.x), "v"(v.y), "v"(v.z));
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(r), "v"(v.w));
    return r;
}
// Stream mass 2^(x c - R) (R an integer reference), c = c_hi + c_lo.
__device__ __forceinline__ float r_mass(float x, float chi, float clo, float R) {
    return __builtin_amdgcn_exp2f(fmaf(x, clo, fmaf(x, chi, -R)));
}
// Octave-relative fixed-point mass of x in octave o: 2^(x c - o) * 2^24,
// rounded down (bounded by 2^25 + a few units: x c may round across o + 1).
__device__ __forceinline__ uint32_t r_fm(float x, float chi, float clo, int o) {
    const float f = fmaf(x, clo, fmaf(x, chi, -(float)o));
    return (uint32_t)(__builtin_amdgcn_exp2f(f) * 16777216.0f);
}
// Stable descending order of sampler.rs:140 as one key: value, then index.
__device__ __forceinline__ unsigned long long r_key(float x, uint32_t idx) {
    return ((unsigned long long)key32(x) << 32) | (uint32_t)~idx;
}

template <int MODE>
__device__ __forceinline__ bool resident_eligible(const RowArgs a, int row) {
    if (a.V < 256 || a.V > kRMaxV) return false;
    if (MODE == kResGreedy || MODE == kResGreedyPen) {
        if (!(a.temperature <= 0.0f)) return false;
        if (MODE == kResGreedyPen) return true;  // any history (its length is checked inside)
    } else {
        if (!(a.temperature > 0.0f) || (a.top_k > 0 && a.top_k < (uint64_t)a.V)) return false;
        if (!(a.top_p >= 1.0f)) return false;
        if (MODE == kResAllPen) return true;
    }
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1) && g1 > g0) return false;
    return true;
}

// Returns NIS_REJECT_NONE when the row is done, else (uniformly across the
// workgroup) why the general path must recompute it; nothing has been
// written then.
//
// kResGreedyPen: greedy with a repetition-penalty history.  The history goes
// into LDS bitmaps before the stream (penalty_bits.h); in a chunk holding
// penalised elements their owner lanes take them out of the register max
// (-inf in their place) and keep the largest penalised value in f64
// (sampler.rs:94-98) with its first index; the two maxima are merged at the
// end, equal values going to the lower index (sampler.rs:172-181).
template <int MODE>
__device__ __forceinline__ uint32_t resident_row(const RowArgs a, const int row, ResShared& sh) {
    constexpr bool GREEDY = MODE == kResGreedy || MODE == kResGreedyPen;
    constexpr bool ALL = MODE == kResAll || MODE == kResAllPen;
    constexpr bool PEN = MODE == kResGreedyPen || MODE == kResAllPen;
    const int l = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int V = (int)a.V;
    const gfp rowp = (gfp)(a.logits + (int64_t)row * a.ld);
    const int mis = (int)(((uintptr_t)rowp >> 2) & 3);  // elements before the row in its 16 B block
    const gf4p base = (gf4p)(rowp - mis);
    const int f_lo = mis ? 1 : 0;          // first float4 slot lying fully inside the row
    const int f_hi = (V + mis - 4) >> 2;   // last one
    const int nsl = (V + mis + 3) >> 2;    // slots touching the row
    const int cpw = (((nsl + 63) >> 6) + kRW - 1) / kRW;  // chunks per wave
    const int wbase = 64 * cpw * w;
    const int Kw = min(max((nsl - wbase + 63) >> 6, 0), cpw);
    const int slot0 = wbase + l;
    // row index of element q of chunk k of this lane
#define NIS_RIDX(k, q) (4 * (slot0 + 64 * (k)) + (q) - mis)

    // the (at most 3 + 3) elements of partial head / tail slots, by one
    // vector load (lane i < 3: element i, lane 3 + i: element V - 6 + 3 + i)
    const float hv = rowp[(l < 3) ? l : ((l < 6) ? V - 6 + l : 0)];
    __builtin_amdgcn_sched_barrier(0);
    const uint64_t bptr = (uint64_t)(uintptr_t)base;
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    f4v xv[kRN];
    xv[0] = nis_buffer_load_f4(rsrc, (Kw > 0) ? 16 * max(slot0, f_lo) : 0x7FFFFFF0, 0, 2);
    __builtin_amdgcn_sched_barrier(0);
    // PEN: the raw history ids (behind chunk 0), and the bitmaps cleared
    const int tid = (int)threadIdx.x;
    uint32_t hid[kPHist / kPB];
    bool hlong = false;  // (the same in every lane) a history too long: the row is declined
    if constexpr (PEN) {
        hlong = pen_load_ids(a, row, tid, hid);
        pen_clear(sh.pb, tid);
    }
    const int voff = 16 * slot0;
#define NIS_RLOAD(k)                                                                          \
    do {                                                                                      \
        xv[k] = nis_buffer_load_f4(rsrc, ((k) < Kw) ? voff + 1024 * (k) : 0x7FFFFFF0, 0, 2);  \
    } while (0)
#pragma unroll
    for (int k = 1; k < kRD && k < kRN; ++k) {
        NIS_RLOAD(k);
        __builtin_amdgcn_sched_barrier(0);  // chunk order = issue order
    }
    typedef const __attribute__((address_space(1))) uint64_t* gu64p;
    uint64_t rsv = 0;
    if (!GREEDY && w == 0) rsv = ((gu64p)(a.rng + 4 * (int64_t)row))[l & 3];
    // PEN: bit k of pany: chunk k of this wave holds a penalised element;
    // bits 4k..4k+3 of pnl: which elements of this lane's slot in chunk k
    uint32_t pany = 0u;
    uint64_t pnl = 0ull;
    if constexpr (PEN) {
        lds_barrier();
        pen_set_bits(sh.pb, hid, V, mis);
        lds_barrier();
        pen_masks<kRN>(sh.pb, wbase, Kw, l, pany, pnl);
    }
    // the CU serves the waves' loads in wave order: later waves run at a
    // higher priority until their stream ends
    __builtin_amdgcn_s_setprio(0);
    if (w >= kRW / 4) __builtin_amdgcn_s_setprio(1);
    if (w >= kRW / 2) __builtin_amdgcn_s_setprio(2);
    if (w >= 3 * kRW / 4) __builtin_amdgcn_s_setprio(3);

    const bool edge_wave = (wbase < f_lo) || (wbase + 64 * Kw - 1 > f_hi);
    const float h0 = bcast_f32(hv, 0), h1 = bcast_f32(hv, 1), h2 = bcast_f32(hv, 2);
    const float t0 = bcast_f32(hv, 3), t1 = bcast_f32(hv, 4), t2 = bcast_f32(hv, 5);
    const f4v ninf4 = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#define NIS_RFIX(k)                                                                           \
    do {                                                                                      \
        if ((k) >= Kw) xv[k] = ninf4;                                                         \
        else if (edge_wave) {                                                                 \
            const int fb0 = wbase + (k) * 64;                                                 \
            if (fb0 < f_lo || fb0 + 63 > f_hi)                                                \
                xv[k] = fix_slot(xv[k], slot0 + (k) * 64, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2); \
        }                                                                                     \
    } while (0)

    // The wave reference follows the wave's running max: when a chunk holds
    // an element more than one octave above it, it moves up to that max and
    // the wave's mass sum is rescaled by the exact power of two.  Masses near
    // the max (the ones that matter) then always have a small argument.
#define NIS_RESCALE(m4, MXR)                                                   \
    if (__ballot((m4) * chi > Rz + 1.0f)) {                                    \
        const float Rn_ = ceilf(wmax_f32(MXR) * chi);                          \
        if (fabsf(Rn_) < 1e30f) {                                              \
            z = ldexp(z, (int)(Rz - Rn_));                                     \
            Rz = Rn_;                                                          \
        }                                                                      \
    }

    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const double c64 = 1.4426950408889634 / temp;            // log2(e) / T
    // c_hi rounded toward zero, so c_lo >= 0 and x = -inf gives -inf, not NaN
    float chi = (float)c64;
    if ((double)chi > c64) chi = __uint_as_float(__float_as_uint(chi) - 1u);
    const float clo = (float)(c64 - (double)chi);

    // =====================================================================
    if constexpr (GREEDY) {
        // ---- greedy: first index of the maximum (sampler.rs:172-181) ----
        float bx = -INFINITY;
        int bi = 0x7FFFFFFF;
        float fs = 0.0f;  // NaN probe: a NaN element makes it NaN (so may +inf beside -inf)
        double py = -INFINITY;  // PEN: this lane's largest penalised value
        int pi = 0x7FFFFFFF;    //   and its first index
        const double pen = (double)a.penalty;
#pragma unroll
        for (int k = 0; k < kRN; ++k) {
            if (k + kRD < kRN) NIS_RLOAD(k + kRD);
            __builtin_amdgcn_sched_barrier(0);
            if (k >= Kw) continue;
            NIS_RFIX(k);
            if constexpr (PEN) {
                if ((pany >> k) & 1u) {
                    const uint32_t nb = (uint32_t)(pnl >> (4 * k)) & 15u;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if ((nb >> q) & 1u) {
                            const double y = pen_value(xv[k][q], pen);
                            const int idx = NIS_RIDX(k, q);
                            if (y != y) fs = NAN;
                            // a -inf value is never recorded: like a plain
                            // -inf it exceeds nothing (sampler.rs:176), so an
                            // all -inf row still returns index 0
                            if (y > py || (y == py && y > -INFINITY && idx < pi)) {
                                py = y;
                                pi = idx;
                            }
                            xv[k][q] = -INFINITY;
                        }
                    }
                }
            }
            const f4v x = xv[k];
            fs += (x.x + x.y) + (x.z + x.w);
            const float m4 = r_max4(x);
            const int q = (x.x == m4) ? 0 : ((x.y == m4) ? 1 : ((x.z == m4) ? 2 : 3));
            const bool up = m4 > bx;
            bi = up ? NIS_RIDX(k, q) : bi;
            bx = up ? m4 : bx;
        }
        __builtin_amdgcn_s_setprio(0);
        // wave: max, then the lowest index holding it
        const float wm = wmax_f32(bx);
        const int wi = (int)wmin_u32((uint32_t)((bx == wm) ? bi : 0x7FFFFFFF));
        const uint32_t bad = (uint32_t)(__ballot(fs != fs) != 0ull);
        double wy = -INFINITY;  // PEN: the wave's largest penalised value
        uint32_t wpi = 0x7FFFFFFFu;
        if (PEN && pany != 0u) {
            wy = py;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) wy = fmax(wy, __shfl_xor(wy, o));
            wpi = wmin_u32((uint32_t)((py == wy) ? pi : 0x7FFFFFFF));
        }
        if (l == 0) {
            RRec r;
            r.z = wy;
            r.mx = wm;
            r.rw = 0.0f;
            r.thc = __int_as_float(wi);
            r.nc = wpi;
            r.bad = bad;
            r.pad = 0u;
            sh.rec[w] = r;
        }
        lds_barrier();
        const bool rv = l < kRW;
        const RRec rr = sh.rec[rv ? l : 0];
        const uint32_t anybad = (uint32_t)(__ballot(rv & (rr.bad != 0u)) != 0ull);
        if (hlong) return NIS_REJECT_CAPACITY;
        if (anybad) return NIS_REJECT_NONFINITE;
        const float rm = rv ? rr.mx : -INFINITY;
        const float M = wmax_f32(rm);
        int tok = (int)wmin_u32((uint32_t)((rv && rr.mx == M) ? __float_as_int(rr.thc) : 0x7FFFFFFF));
        double Mx = (double)M;
        if constexpr (PEN) {
            // the penalised maximum against the register one: the larger value,
            // on equal values the lower index
            double Y = rv ? rr.z : -INFINITY;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) Y = fmax(Y, __shfl_xor(Y, o));
            const int ty = (int)wmin_u32((rv && rr.z == Y) ? rr.nc : 0x7FFFFFFFu);
            if (Y > Mx) tok = ty;
            else if (Y == Mx) tok = min(tok, ty);
            Mx = fmax(Mx, Y);
        }
        if (tok == 0x7FFFFFFF) tok = 0;  // every element -inf: nothing exceeds work[0]
        if (w == 0 && l == 0) write_row_result(a, row, (uint32_t)tok, NIS_PATH_GREEDY, Mx, 0.0,
                                               0.0, -1.0, 0.0, 0, 1);
        return NIS_REJECT_NONE;
    }

    // ---- wave reference from the first chunk ----------------------------
    NIS_RTDECL
    NIS_RTS(0);
    NIS_RFIX(0);
    float c0m = r_max4(xv[0]);
    if constexpr (PEN) {
        // the penalised elements of chunk 0 by their penalised values (rounded
        // up), so that the reference starts at the wave's values and not
        // above them (the masses' f32 arguments lose precision with depth)
        if (pany & 1u) {
            const uint32_t nb0 = (uint32_t)pnl & 15u;
            f4v t = xv[0];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if ((nb0 >> q) & 1u) t[q] = pen_f32_up(pen_value(xv[0][q], (double)a.penalty));
            c0m = r_max4(t);
        }
    }
    float m0 = wmax_f32(c0m);
    if (m0 == -INFINITY && Kw > 1) {
        // chunk 0 holds nothing above -inf (a masked stretch): the first
        // reference comes from the wave's other chunks (without a penalty,
        // all of them, their loads issued now and again by the stream as
        // usual; with one, the chunks already in flight, which keeps the
        // penalised form within its registers).  A wave still empty there
        // keeps 0, and the reference guard at the first barrier declines the
        // row if that leaves it far above the wave's values.
        constexpr int KREF = PEN ? (kRD < kRN ? kRD : kRN) : kRN;
        if constexpr (!PEN) {
#pragma unroll
            for (int k = kRD; k < kRN; ++k) NIS_RLOAD(k);
        }
        float mw = -INFINITY;
#pragma unroll
        for (int k = 1; k < KREF; ++k) {
            if (k < Kw) {
                f4v t = xv[k];
                if (edge_wave) {
                    const int fb0 = wbase + k * 64;
                    if (fb0 < f_lo || fb0 + 63 > f_hi)
                        t = fix_slot(t, slot0 + k * 64, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2);
                }
                // (penalised elements left out: if one of them is the wave's
                // max, the stream raises the reference when it meets it)
                if (PEN && ((pany >> k) & 1u)) {
                    const uint32_t nbk = (uint32_t)(pnl >> (4 * k)) & 15u;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if ((nbk >> q) & 1u) t[q] = -INFINITY;
                }
                mw = fmaxf(mw, r_max4(t));
            }
        }
        m0 = wmax_f32(mw);
    }
    NIS_RTS(1);
    const float Rw = (m0 > -INFINITY && fabsf(m0 * chi) < 1e30f) ? ceilf(m0 * chi) : 0.0f;

    // =====================================================================
    if constexpr (ALL) {
        // ---- top-p off: every element kept ------------------------------
        // (with a penalty, a penalised element keeps its logit in registers
        // and its f64 value's mass in the chunk sums; the max splits into
        // the unpenalised one, the penalised one rounded up, which with it
        // bounds every mass's argument, and the exact penalised one.  Top-p
        // off ranks nothing, so the value may be x * (1/pen): within an ulp
        // of the reference's quotient, far below the masses' own rounding.
        // Its mass is the f32 form of the unpenalised ones, y split as
        // yh + yl, so the walk recomputes it bit for bit.)
        double z = 0.0;
        float mx = -INFINITY;
        float mxp = -INFINITY;    // PEN: largest penalised value, rounded up
        double ymx = -INFINITY;   // PEN: the same, exact
        const double pen = (double)a.penalty, rpen = 1.0 / pen;
        auto pval = [&](float x) -> double { return (x > 0.0f) ? (double)x * rpen : (double)x * pen; };
        float czh = chi, czl = clo, Rz = Rw;
        asm volatile("" : "+v"(czh), "+v"(czl));
        auto pmass = [&](double y, float R) -> float {
            const float yh = (float)y, yl = (float)(y - (double)yh);
            return __builtin_amdgcn_exp2f(fmaf(yl, czh, fmaf(yh, czl, fmaf(yh, czh, -R))));
        };
        float s4v[kRN];  // this lane's float4 mass of chunk k, against reference Rk[k]
        float Rk[kRN];
#pragma unroll
        for (int k = 0; k < kRN; ++k) {
            if (k + kRD < kRN) NIS_RLOAD(k + kRD);
            __builtin_amdgcn_sched_barrier(0);
            s4v[k] = 0.0f;
            Rk[k] = Rz;
            if (k >= Kw) continue;
            if (k > 0) NIS_RFIX(k);
            const f4v x = xv[k];
            f4v xm = x;                // the unpenalised values (-inf for penalised ones)
            uint32_t nb = 0u;          // PEN: penalised elements of this float4
            double yv[4] = {0.0, 0.0, 0.0, 0.0};
            float m4p = -INFINITY;     // PEN: their max, rounded up
            if constexpr (PEN) {
                if ((pany >> k) & 1u) {
                    nb = (uint32_t)(pnl >> (4 * k)) & 15u;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if ((nb >> q) & 1u) {
                            yv[q] = pval(x[q]);
                            xm[q] = -INFINITY;
                            m4p = fmaxf(m4p, pen_f32_up(yv[q]));
                            ymx = fmax(ymx, yv[q]);
                        }
                    }
                    mxp = fmaxf(mxp, m4p);
                }
            }
            const float m4 = r_max4(xm);
            mx = fmaxf(mx, m4);
            NIS_RESCALE(fmaxf(m4, m4p), fmaxf(mx, mxp))
            Rk[k] = Rz;
            float e0 = r_mass(x.x, czh, czl, Rz), e1 = r_mass(x.y, czh, czl, Rz);
            float e2 = r_mass(x.z, czh, czl, Rz), e3 = r_mass(x.w, czh, czl, Rz);
            if constexpr (PEN) {
                if ((pany >> k) & 1u) {
                    if (nb & 1u) e0 = pmass(yv[0], Rz);
                    if (nb & 2u) e1 = pmass(yv[1], Rz);
                    if (nb & 4u) e2 = pmass(yv[2], Rz);
                    if (nb & 8u) e3 = pmass(yv[3], Rz);
                }
            }
            const float s4 = (e0 + e1) + (e2 + e3);
            s4v[k] = s4;
            z += (double)s4;
        }
        __builtin_amdgcn_s_setprio(0);
        mx = wmax_f32(mx);
        z = wsum_f64(z);
        if constexpr (PEN) {
            mxp = wmax_f32(mxp);
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ymx = fmax(ymx, __shfl_xor(ymx, o));
            if (l == 0) {
                sh.pmx[w] = mxp;
                sh.pymx[w] = ymx;
            }
        }
        // with stats: the elements above -inf (every one of them is kept)
        uint32_t nfin = 0u;
        if (a.stats) {
#pragma unroll
            for (int k = 0; k < kRN; ++k)
                if (k < Kw)
                    nfin += (uint32_t)(xv[k].x > -INFINITY) + (uint32_t)(xv[k].y > -INFINITY) +
                            (uint32_t)(xv[k].z > -INFINITY) + (uint32_t)(xv[k].w > -INFINITY);
            nfin = wsum_u32(nfin);
        }
        if (l == 0) {
            RRec r;
            r.z = z;
            r.mx = mx;
            r.rw = Rz;
            r.thc = 0.0f;
            r.nc = nfin;
            r.bad = (uint32_t)!(z < INFINITY);
            r.pad = 0u;
            sh.rec[w] = r;
        }
        uint64_t rst = 0;
        if (w == 0) {
            uint64_t st[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                st[j] = ((uint64_t)bcast_u32((uint32_t)(rsv >> 32), j) << 32) | bcast_u32((uint32_t)rsv, j);
            const double u0 = rng_next_f64(st);
            if (l == 0) sh.u0 = u0;
            rst = (l == 0) ? st[0] : (l == 1) ? st[1] : (l == 2) ? st[2] : st[3];
        }
        lds_barrier();
        if (hlong) return NIS_REJECT_CAPACITY;
        const bool rv = l < kRW;
        const RRec rr = sh.rec[rv ? l : 0];
        // M bounds every element's x c (with a penalty, the penalised values
        // rounded up); Mx is the exact row max, for the statistics
        float M = wmax_f32(rv ? rr.mx : -INFINITY);
        double Mx = (double)M;
        const float pm = (PEN && rv) ? sh.pmx[l] : -INFINITY;
        if constexpr (PEN) {
            double py = rv ? sh.pymx[l] : -INFINITY;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) py = fmax(py, __shfl_xor(py, o));
            Mx = fmax(Mx, py);
            M = fmaxf(M, wmax_f32(pm));
        }
        const float R = (M > -INFINITY && fabsf(M * chi) < 1e30f) ? ceilf(M * chi) : 0.0f;
        // each wave's total in 2^R units (exact power-of-two rescales; a wave
        // more than ~1075 octaves below R holds 0 in f64, as its exp(w - max)
        // does in the reference's, and is never drawn)
        const double T = rv ? ldexp(rr.z, (int)fmaxf(rr.rw - R, -2048.0f)) : 0.0;
        const double Tincl = rscan16_f64(T);
        const double Z = bcast_f64(Tincl, 15);
        // a wave's reference only rises during the stream: one that ended
        // more than 8 octaves above the wave's max would cost its masses
        // precision (their f32 arguments' rounding grows with depth: 8
        // octaves, 3e-7) or, past 64 octaves, the masses themselves; that is
        // harmless only for a wave whose max lies 20 or more octaves below R
        // (the first reference is the wave's own max, so this is a guard)
        const float wtop = rv ? fmaxf(rr.mx, pm) : -INFINITY;
        const float cw = ceilf(wtop * chi);
        const bool gapbad = rv & (wtop > -INFINITY) & (rr.rw - cw > 8.0f) &
                            ((R - cw < 20.0f) | (rr.rw - cw > 64.0f));
        const bool ok = (M > -INFINITY) & (M < INFINITY) & (Z > 0.0) & (Z < INFINITY) &
                        (__ballot(rv & (rr.bad != 0u)) == 0ull) & (__ballot(gapbad) == 0ull);
        if (!ok) return NIS_REJECT_NONFINITE;
        if (w == 0 && l < 4) a.rng[4 * (int64_t)row + l] = rst;
        const double u = sh.u0;
        const double r = u * Z;
        // the chosen wave: the first whose inclusive total reaches r (the
        // last with mass if rounding leaves r above every prefix)
        const uint64_t hw = __ballot(rv & (T > 0.0) & (Tincl >= r));
        const uint64_t nzw = __ballot(rv & (T > 0.0));
        const int ws = hw ? (__ffsll((long long)hw) - 1) : (63 - __clzll((long long)nzw));
        if (w != ws) return NIS_REJECT_NONE;
        const uint32_t nkept = a.stats ? wsum_u32(rv ? rr.nc : 0u) : 0u;
        // r inside this wave, in 2^R_w units
        const double rw_ = ldexp(r - bcast_f64(Tincl - T, ws), (int)(R - Rz));
        // chunk totals (2^Rz units, exact rescales): a transposed sum of the
        // per-lane chunk masses
        float* const s4w = &sh.s4[w][0][0];
#pragma unroll
        for (int k = 0; k < kRN; ++k) s4w[k * 64 + l] = ldexpf(s4v[k], (int)(Rk[k] - Rz));
        lds_wave_fence();
        // lane j < 4 kRN: quarter j & 3 of chunk j >> 2
        double qs = 0.0;
        if (l < 4 * kRN) {
            const int kk = l >> 2, qq = l & 3;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f4v v = *reinterpret_cast<const f4v*>(&s4w[kk * 64 + 16 * qq + i]);
                qs += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
            }
        }
        {
            const uint64_t b_ = (uint64_t)__double_as_longlong(qs);
            const uint64_t lo_ = dpp0<0x111, 0xF>((uint32_t)b_), hi_ = dpp0<0x111, 0xF>((uint32_t)(b_ >> 32));
            qs += __longlong_as_double((long long)((hi_ << 32) | lo_));   // lanes 4i+1: quarters 0+1, 4i+3: 2+3
        }
        {
            const uint64_t b_ = (uint64_t)__double_as_longlong(qs);
            const uint64_t lo_ = dpp0<0x112, 0xF>((uint32_t)b_), hi_ = dpp0<0x112, 0xF>((uint32_t)(b_ >> 32));
            qs += __longlong_as_double((long long)((hi_ << 32) | lo_));   // lane 4i+3: the chunk
        }
        // chunk k's total sits in lane 4k + 3; gather them into lanes 0..kRN-1
        const double ck = __shfl(qs, 4 * min(l, kRN - 1) + 3);
        const double cks = (l < kRN && l < Kw) ? ck : 0.0;
        const double cincl = rscan16_f64(cks);  // kRN <= 16: one DPP row
        const uint64_t hk = __ballot((l < 16) & (cks > 0.0) & (cincl >= rw_));
        const uint64_t nzk = __ballot((l < 16) & (cks > 0.0));
        const int kc = hk ? (__ffsll((long long)hk) - 1) : (63 - __clzll((long long)(nzk | 1ull)));
        const double rk_ = rw_ - bcast_f64(cincl - cks, kc);
        // lanes of chunk kc in index order
        f4v xc = xv[0];
        float sc = s4v[0], Rc = Rk[0];
#pragma unroll
        for (int k = 1; k < kRN; ++k)
            if (k == kc) {
                xc = xv[k];
                sc = s4v[k];
                Rc = Rk[k];
            }
        const int dc = (int)(Rc - Rz);
        const double sl = (double)ldexpf(sc, dc);
        const double lincl = wscan_f64(sl);
        const uint64_t hl = __ballot((sl > 0.0) & (lincl >= rk_));
        const uint64_t nzl = __ballot(sl > 0.0);
        const int lc = hl ? (__ffsll((long long)hl) - 1) : (63 - __clzll((long long)(nzl | 1ull)));
        if (l == lc) {
            double run = rk_ - (lincl - sl);
            float ev[4] = {ldexpf(r_mass(xc.x, czh, czl, Rc), dc), ldexpf(r_mass(xc.y, czh, czl, Rc), dc),
                           ldexpf(r_mass(xc.z, czh, czl, Rc), dc), ldexpf(r_mass(xc.w, czh, czl, Rc), dc)};
            double vq[4] = {(double)xc.x, (double)xc.y, (double)xc.z, (double)xc.w};  // values after the penalty
            if constexpr (PEN) {
                // the penalised elements' masses exactly as the stream summed them
                const uint32_t nbc = (uint32_t)(pnl >> (4 * kc)) & 15u;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if ((nbc >> q) & 1u) {
                        vq[q] = pval(xc[q]);
                        ev[q] = ldexpf(pmass(vq[q], Rc), dc);
                    }
                }
            }
            // the first element whose running mass reaches r (the last with
            // mass if rounding leaves r above them all)
            int q = -1, qlast = 0;
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                if (ev[qq] > 0.0f) {
                    qlast = qq;
                    if (q < 0) {
                        run -= (double)ev[qq];
                        if (run <= 0.0) q = qq;
                    }
                }
            }
            if (q < 0) q = qlast;
            const double xq = vq[q];
            uint32_t tok = (uint32_t)NIS_RIDX(kc, q);
            if (u == 0.0) tok = 0u;  // r == 0 stops the reference's walk at index 0
            emit_token(a, row, tok);
            if (a.stats) {
                // the drawn token's mass against the row max, exactly reduced
                const double em = exp2(xq * c64 - Mx * c64);
                const double zM = Z * exp2((double)R - Mx * c64);  // (R - Mx c within about [0, 1])
                write_row_stats(a, row, tok, NIS_PATH_DRAW, Mx / temp, zM, 0.0, u,
                                (u == 0.0) ? 0.0 : em / zM, (uint64_t)nkept, 1);
            }
        }
        return NIS_REJECT_NONE;
    }

    return NIS_REJECT_NONE;  // (no other mode)
#undef NIS_RLOAD
#undef NIS_RFIX
#undef NIS_RIDX
#undef NIS_RESCALE
}

// One 1024-lane workgroup per row: the resident path in the launch's MODE,
// the general path (on the first 512 lanes) for a row it declines or cannot
// take.
template <int MODE>
__global__ __launch_bounds__(kRB) void sample_rows_resident_kernel(RowArgs a) {
    __shared__ union {
        GeneralShared g;
        ResShared r;
    } sh;
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;  // a finished sequence (decode step)
    asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.temperature), "s"(a.top_p),
                 "s"(a.penalty), "s"(a.gen_ids), "s"(a.gen_off));
    uint32_t reject = NIS_REJECT_SHAPE;
    if (resident_eligible<MODE>(a, row)) {
        reject = resident_row<MODE>(a, row, sh.r);
        if (reject == NIS_REJECT_NONE) return;
    }
    if (threadIdx.x >= kBlock) return;
    __syncthreads();
    general_row<1>(a, row, sh.g, reject);
}

}  // namespace nis
