// resident_path.h — one row per 1024-lane workgroup (16 wave64s, four per
// SIMD), the row held in VGPRs (V <= 53245): the hot path of
// nis_sample_batch for greedy rows, top-p off and top-p rows whose nucleus
// is a small share of the vocabulary (src/sampler.rs:163-217).
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
// reference of the wave (R_w, from its first chunk) and masses are f32,
// summed in f64: the row total Z and the per-wave totals.  Candidates of the
// top-p cutoff get exact fixed-point masses instead: bucket b = floor(64 t)
// of t = f32(x c_hi) (monotone in x), octave o = b >> 6, and
// fm = 2^f * 2^24 rounded down, f = fma(x, c_lo, fma(x, c_hi, -o)) (the
// fraction, computed without cancellation), so fm << (o - R + 16) is the
// mass in units of 2^(R - 40) with a relative error of ~1e-7 at any depth.
//
// Sparse top-p (sampler.rs:118-160) without a sort.  The reference keeps
// sorted position pos iff D(pos) = cum_excl(pos) - q(pos) <= p Z; D is
// non-decreasing in pos, so the kept set is a prefix of the stable order.
//   Stream.  Each wave histograms the float4 maxima of its first kRS chunks
//   (1/8-octave bins) and takes thc_w, the lower edge of the top bins holding
//   at most kRTop of those 256 maxima; it publishes thc_w (an LDS max) and
//   lists every float4 holding an element >= thl = max(thc_w, the published
//   maximum so far) in an LDS ring.  Every 64 listed float4s, the wave turns
//   them into candidates (elements >= thl) one entry per lane: the
//   candidate's bucket and fm join a shared histogram of buckets (count << 48
//   | sum of fm) and one of octaves, and the candidate is appended to the
//   wave's record list (value, index, bucket, fm) in index order.  So the
//   histogram is complete when the stream ends.
//   Every element >= x_lo = max_w thc_w is a candidate of its wave, so the
//   buckets from blo = 64 x_lo up are complete.
//   Cutoff (every wave, the same data and instructions).  With G(b) the mass
//   of the buckets above b and m_up(b) a bound of any mass in b, b_p is the
//   deepest non-empty bucket with G(b) - m_up(b) <= p Z.  Everything below it
//   is removed, everything above kept (the last element y of the next
//   non-empty bucket above has D(y) <= G(b_p) - 2 m(y) < p Z), and the cutoff
//   lies among b_p's members, ranked exactly (descending value, ascending
//   index) against sampler.rs:150.  G(blo - 1) - m_up(blo - 1) > p Z proves
//   that nothing below blo is kept.
//   After the one barrier that ends the stream, each wave sums its kept
//   records above b_p and lists its members of b_p; after a second barrier
//   every wave ranks the members, and the wave holding the draw walks its
//   records (sampler.rs:209-216).  Kept masses are exact integers (u64), so
//   the totals and the walk agree to the last bit.
// Top-p off: every element is kept; the walk goes waves -> chunks -> lanes
// -> elements over the stream's own f32 masses (chunk totals from one
// transposed LDS sum in the chosen wave), and the drawn token's probability
// uses its exact mass.
// Greedy (sampler.rs:172-181): the first index of the maximum.
//
// Any row this path cannot prove (non-finite values, a threshold above the
// cutoff, list or bucket overflow, a kept range deeper than 16 octaves)
// returns a reject code before anything is written, and the caller runs the
// general path on it.
#pragma once
#include "fast_path.h"

namespace nis {

constexpr int kRB = 1024;                  // lanes per workgroup
constexpr int kRW = kRB / 64;              // waves per workgroup
constexpr int kRN = 13;                    // float4 chunks per lane (at most)
constexpr int kRMaxV = kRB * 4 * kRN - 3;  // 53245
constexpr int kRD = 3;                     // loads in flight per lane ahead of the one in use
constexpr int kRS = 4;                     // sample chunks per wave
constexpr uint32_t kRTop = 44;             // sampled float4 maxima allowed above thc_w
constexpr int kRQ = 128;                   // listed float4s awaiting their round (ring, per wave)
constexpr int kRC = 256;                   // candidate records per wave
constexpr int kRRes = 64;                  // buckets per octave
constexpr int kRLog = 6;
constexpr int kRHB = 32 * kRRes;           // bucket ring: 32 octaves
constexpr int kRMem = 64;                  // members of the cutoff bucket
constexpr int kRDeep = 16;                 // kept octaves below R (exact fixed point)

enum { kResSparse = 0, kResAll = 1, kResGreedy = 2 };

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

// A candidate: its logit, row index, bucket and octave-relative mass.
struct alignas(16) RCand {
    float x;
    uint32_t idx;
    int32_t b;
    uint32_t fm;
};
// Stream-end record of one wave (lane 0 writes it).
struct alignas(16) RRec {
    double z;      // sum of 2^(x c - R_w) over the wave's elements (greedy: unused)
    float mx;      // wave max logit
    float rw;      // R_w
    float thc;     // sample threshold in x c units (-inf: no data); greedy: best index
    uint32_t nc;   // candidate records (> kRC: overflow)
    uint32_t bad;  // the wave saw input this path does not take
    uint32_t pad;
};

// The cutoff (wave 0 writes it between barriers).
struct alignas(16) RCut {
    unsigned long long gp;  // G(b_p): mass of the buckets above b_p, 2^(R - 40) units
    double pz;              // p Z, the same units
    double zr;              // Z, 2^R units
    float M;                // row max
    float R;                // ceil(M c)
    int32_t bp;             // b_p
    uint32_t nsel;          // candidates in b_p
    uint32_t rej;           // NIS_REJECT_*
    uint32_t nab;           // candidates above b_p
    uint32_t pad[2];
};
// One wave's records after the cutoff: kept mass above b_p and count.
struct alignas(16) RAbove {
    unsigned long long m;
    uint32_t n;
    uint32_t pad;
};

struct ResShared {
    union {
        struct {
            f4v q[kRW][kRQ];             // listed float4s, ring per wave
            uint16_t qpos[kRW][kRQ];     //   chunk * 64 + lane
            union {
                RCand cand[kRW][kRC];    // candidates, index order per wave
                uint32_t whist[kRW][256 * 4];  // (before them) each wave's sample histogram
            } c;
        } s;
        float s4[kRW][kRN][64];          // top-p off: per-chunk per-lane f32 masses
    } u;
    unsigned long long hist[kRHB];       // [b & (kRHB-1)]: count << 48 | sum of fm
    unsigned long long oct[32];          // the same per octave
    RCand mem[kRMem];                    // members of b_p
    RRec rec[kRW];
    RCut cut;
    RAbove above[kRW];
    unsigned long long otot[32];         // cutoff search: octave oM - j's total (2^(R - 40) units)
    unsigned long long opass[kRW][2];    // each wave's deepest passing bucket (as u64) and G       // per-wave kept mass above b_p (2^(R-40) units)
    double u0;                           // the draw
    uint32_t nmem;
    uint32_t kxlo;                       // running max of the published thresholds (key32)
    // the waves' stream-end figures, reduced as they arrive (order-preserving keys)
    uint32_t kmax;                       // row max
    uint32_t krw;                        // lowest reference of a wave with data
    uint32_t kth;                        // lowest threshold of a wave with candidates
    uint32_t knc;                        // most candidate records of a wave
    uint32_t kbad;                       // a wave saw input this path does not take
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
// Bucket floor(64 f32(x c_hi)): monotone in x.
__device__ __forceinline__ int r_bucket(float x, float chi) {
    int b;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(b) : "v"((x * chi) * (float)kRRes));
    return b;
}
// Octave-relative fixed-point mass of x in octave o: 2^(x c - o) * 2^24,
// rounded down (bounded by 2^25 + a few units: x c may round across o + 1).
__device__ __forceinline__ uint32_t r_fm(float x, float chi, float clo, int o) {
    const float f = fmaf(x, clo, fmaf(x, chi, -(float)o));
    return (uint32_t)(__builtin_amdgcn_exp2f(f) * 16777216.0f);
}
// fm in octave o as an integer in 2^(R - 40) units (o >= R - 16 exact; a
// deeper octave is truncated, which only ever lowers a sum).
__device__ __forceinline__ unsigned long long r_u40(unsigned long long fm, int o, int R) {
    const int sh = o - R + 16;
    return sh >= 0 ? (fm << (uint32_t)min(sh, 63)) : (fm >> (uint32_t)min(-sh, 63));
}
// Upper bound of one element's mass in bucket b (its upper edge, inflated
// for the roundings of x c and exp2), 2^(R - 40) units, as f64.
__device__ __forceinline__ double r_mup(int b, int R) {
    return ldexp((double)__builtin_amdgcn_exp2f((float)((b + 1) & (kRRes - 1)) * (1.0f / kRRes)) *
                     1.0001,
                 ((b + 1) >> kRLog) - R + 40);
}
// Stable descending order of sampler.rs:140 as one key: value, then index.
__device__ __forceinline__ unsigned long long r_key(float x, uint32_t idx) {
    return ((unsigned long long)key32(x) << 32) | (uint32_t)~idx;
}

template <int MODE>
__device__ __forceinline__ bool resident_eligible(const RowArgs a, int row) {
    if (a.V < 256 || a.V > kRMaxV) return false;
    if (MODE == kResGreedy) {
        if (!(a.temperature <= 0.0f)) return false;
    } else {
        if (!(a.temperature > 0.0f) || (a.top_k > 0 && a.top_k < (uint64_t)a.V)) return false;
        if (MODE == kResAll ? !(a.top_p >= 1.0f) : !(a.top_p > 0.0f && a.top_p < 1.0f)) return false;
    }
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1) && g1 > g0) return false;
    return true;
}

// Returns NIS_REJECT_NONE when the row is done, else (uniformly across the
// workgroup) why the general path must recompute it; nothing has been
// written then.
template <int MODE>
__device__ __forceinline__ uint32_t resident_row(const RowArgs a, const int row, ResShared& sh) {
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
    if (MODE == kResSparse) {
        *reinterpret_cast<u4v*>(&sh.hist[w * (kRHB / kRW) + 2 * l]) = u4v{0u, 0u, 0u, 0u};
        if (l < 32 / kRW) sh.oct[w * (32 / kRW) + l] = 0ull;
        if (w == 0 && l == 0) {
            sh.nmem = 0u;
            sh.kxlo = 0u;
            sh.kmax = 0u;
            sh.krw = 0xFFFFFFFFu;
            sh.kth = 0xFFFFFFFFu;
            sh.knc = 0u;
            sh.kbad = 0u;
        }
        lds_barrier();
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
    if (MODE != kResGreedy && w == 0) rsv = ((gu64p)(a.rng + 4 * (int64_t)row))[l & 3];
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
#define NIS_RESCALE(m4)                                                        \
    if (__ballot((m4) * chi > Rz + 1.0f)) {                                    \
        const float Rn_ = ceilf(wmax_f32(mx) * chi);                           \
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
    if constexpr (MODE == kResGreedy) {
        // ---- greedy: first index of the maximum (sampler.rs:172-181) ----
        float bx = -INFINITY;
        int bi = 0x7FFFFFFF;
        float fs = 0.0f;  // NaN probe: a NaN element makes it NaN (so may +inf beside -inf)
#pragma unroll
        for (int k = 0; k < kRN; ++k) {
            if (k + kRD < kRN) NIS_RLOAD(k + kRD);
            __builtin_amdgcn_sched_barrier(0);
            if (k >= Kw) continue;
            NIS_RFIX(k);
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
        if (l == 0) {
            RRec r;
            r.z = 0.0;
            r.mx = wm;
            r.rw = 0.0f;
            r.thc = __int_as_float(wi);
            r.nc = 0u;
            r.bad = bad;
            r.pad = 0u;
            sh.rec[w] = r;
        }
        lds_barrier();
        const bool rv = l < kRW;
        const RRec rr = sh.rec[rv ? l : 0];
        const uint32_t anybad = (uint32_t)(__ballot(rv & (rr.bad != 0u)) != 0ull);
        if (anybad) return NIS_REJECT_NONFINITE;
        const float rm = rv ? rr.mx : -INFINITY;
        const float M = wmax_f32(rm);
        int tok = (int)wmin_u32((uint32_t)((rv && rr.mx == M) ? __float_as_int(rr.thc) : 0x7FFFFFFF));
        if (tok == 0x7FFFFFFF) tok = 0;  // every element -inf: nothing exceeds work[0]
        if (w == 0 && l == 0) write_row_result(a, row, (uint32_t)tok, NIS_PATH_GREEDY, (double)M, 0.0,
                                               0.0, -1.0, 0.0, 0, 1);
        return NIS_REJECT_NONE;
    }

    // ---- wave reference from the first chunk ----------------------------
    NIS_RTDECL
    NIS_RTS(0);
    NIS_RFIX(0);
    const float m0 = wmax_f32(r_max4(xv[0]));
    NIS_RTS(1);
    const float Rw = (m0 > -INFINITY && fabsf(m0 * chi) < 1e30f) ? ceilf(m0 * chi) : 0.0f;

    // =====================================================================
    if constexpr (MODE == kResAll) {
        // ---- top-p off: every element kept ------------------------------
        double z = 0.0;
        float mx = -INFINITY;
        float czh = chi, czl = clo, Rz = Rw;
        asm volatile("" : "+v"(czh), "+v"(czl));
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
            const float m4 = r_max4(x);
            mx = fmaxf(mx, m4);
            NIS_RESCALE(m4)
            Rk[k] = Rz;
            const float e0 = r_mass(x.x, czh, czl, Rz), e1 = r_mass(x.y, czh, czl, Rz);
            const float e2 = r_mass(x.z, czh, czl, Rz), e3 = r_mass(x.w, czh, czl, Rz);
            const float s4 = (e0 + e1) + (e2 + e3);
            s4v[k] = s4;
            z += (double)s4;
        }
        __builtin_amdgcn_s_setprio(0);
        mx = wmax_f32(mx);
        z = wsum_f64(z);
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
        const bool rv = l < kRW;
        const RRec rr = sh.rec[rv ? l : 0];
        const float M = wmax_f32(rv ? rr.mx : -INFINITY);
        const float R = (M > -INFINITY && fabsf(M * chi) < 1e30f) ? ceilf(M * chi) : 0.0f;
        const float rwmin = -wmax_f32(rv && rr.mx > -INFINITY ? -rr.rw : -INFINITY);
        // each wave's total in 2^R units (exact power-of-two rescales)
        const double T = rv ? ldexp(rr.z, (int)(rr.rw - R)) : 0.0;
        const double Tincl = rscan16_f64(T);
        const double Z = bcast_f64(Tincl, 15);
        const bool ok = (M > -INFINITY) & (M < INFINITY) & (Z > 0.0) & (Z < INFINITY) &
                        (__ballot(rv & (rr.bad != 0u)) == 0ull) & (fmaf(M, chi, -rwmin) <= 100.0f);
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
        float* const s4w = &sh.u.s4[w][0][0];
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
            const float ev[4] = {ldexpf(r_mass(xc.x, czh, czl, Rc), dc), ldexpf(r_mass(xc.y, czh, czl, Rc), dc),
                                 ldexpf(r_mass(xc.z, czh, czl, Rc), dc), ldexpf(r_mass(xc.w, czh, czl, Rc), dc)};
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
            const float xq = elem(xc, q);
            uint32_t tok = (uint32_t)NIS_RIDX(kc, q);
            if (u == 0.0) tok = 0u;  // r == 0 stops the reference's walk at index 0
            emit_token(a, row, tok);
            if (a.stats) {
                // the drawn token's mass against the row max, exactly reduced
                const double em = exp2((double)xq * c64 - (double)M * c64);
                const double zM = ldexp(Z, (int)R) * exp2(-(double)M * c64);
                write_row_stats(a, row, tok, NIS_PATH_DRAW, (double)M / temp, zM, 0.0, u,
                                (u == 0.0) ? 0.0 : em / zM, (uint64_t)nkept, 1);
            }
        }
        return NIS_REJECT_NONE;
    }

    // =====================================================================
    // ---- sparse top-p -----------------------------------------------------
    const float p = a.top_p;
    const float RwH = Rw + 8.0f;  // top of the sample histogram (8 octaves of head room)
    double z = 0.0;
    float mx = -INFINITY;
    float czh = chi, czl = clo, Rz = Rw;
    asm volatile("" : "+v"(czh), "+v"(czl));
    float thc = INFINITY;  // this wave's sample threshold (x c units, a multiple of 1/8)
    float thl = INFINITY;  // its listing threshold: thc raised to the waves' running max
    float thx = INFINITY;  // the same in logit units, rounded down
    uint32_t nq = 0;       // float4s listed (ring position)
    uint32_t np = 0;       // of them turned into candidates
    uint32_t nc = 0;       // candidate records
    float mcs[kRS];
    uint32_t* const whist = &sh.u.s.c.whist[w][0];
    *reinterpret_cast<u4v*>(&whist[4 * l]) = u4v{0u, 0u, 0u, 0u};
    const uint32_t q0 = lds_addr(&sh.u.s.q[w][0]), qp0 = lds_addr(&sh.u.s.qpos[w][0]);
    const uint32_t cand0 = lds_addr(&sh.u.s.c.cand[w][0]);
    const uint32_t hist0 = lds_addr(&sh.hist[0]), oct0 = lds_addr(&sh.oct[0]);

    // list the float4s of chunk k holding an element >= the threshold
#define NIS_RLIST(k, cond)                                                                  \
    {                                                                                       \
        const uint64_t mk = __ballot(cond);                                                 \
        const uint32_t slot = (nq + lane_rank(mk)) & (uint32_t)(kRQ - 1);                   \
        lds_put_x4_u16(mk, q0 + 16 * slot, xv[k], qp0 + 2 * slot, (uint32_t)((k) * 64 + l)); \
        nq += (uint32_t)__popcll(mk);                                                       \
    }
    // One round: lane j takes listed float4 np + j (if listed); its elements
    // >= thl become candidates: histograms and records (index order).
    auto round = [&](uint32_t navail) {
        const uint32_t j = np + (uint32_t)l;
        const bool has = (uint32_t)l < navail;
        lds_wave_fence();
        const uint32_t slot = j & (uint32_t)(kRQ - 1);
        const f4v v = sh.u.s.q[w][slot];
        const uint32_t pos = sh.u.s.qpos[w][slot];
        const int ib = 4 * (wbase + 64 * (int)(pos >> 6) + (int)(pos & 63u)) - mis;
        uint32_t cm = 0u;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) cm |= (has & (elem(v, qq) * chi >= thl)) ? (1u << qq) : 0u;
        const uint32_t cnt = (uint32_t)__popc(cm);
        const uint32_t incl = wscan_u32(cnt);
        const uint32_t cb = nc + incl - cnt;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const bool ok = (cm >> qq) & 1u;
            const uint64_t am = __ballot(ok);
            if (am) {
                const float x = elem(v, qq);
                const int b = r_bucket(x, chi);
                const int o = b >> kRLog;
                const uint32_t fm = r_fm(x, chi, clo, o);
                const uint32_t rs = cb + (uint32_t)__popc(cm & ((1u << qq) - 1u));
                lds_add_u64x2(am, hist0 + 8 * ((uint32_t)b & (uint32_t)(kRHB - 1)),
                              oct0 + 8 * ((uint32_t)o & 31u), (1ull << 48) | (uint64_t)fm);
                const uint64_t wm = __ballot(ok & (rs < (uint32_t)kRC));
                lds_put_b128_m(wm, cand0 + 16 * min(rs, (uint32_t)kRC - 1),
                               u4v{__float_as_uint(x), (uint32_t)(ib + qq), (uint32_t)b, fm});
            }
        }
        nc += (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
        np += min(navail, 64u);
    };

#pragma unroll
    for (int k = 0; k < kRN; ++k) {
        if (k + kRD < kRN) NIS_RLOAD(k + kRD);
        __builtin_amdgcn_sched_barrier(0);
        if (k >= Kw && k >= kRS) continue;
        if (k > 0) NIS_RFIX(k);
        const f4v x = xv[k];
        const float m4 = r_max4(x);
        mx = fmaxf(mx, m4);
        NIS_RESCALE(m4)
        const float e0 = r_mass(x.x, czh, czl, Rz), e1 = r_mass(x.y, czh, czl, Rz);
        const float e2 = r_mass(x.z, czh, czl, Rz), e3 = r_mass(x.w, czh, czl, Rz);
        z += (double)((e0 + e1) + (e2 + e3));
        if (k < kRS) {
            const float mc = m4 * chi;
            mcs[k] = mc;
            const float tb = floorf((RwH - mc) * 8.0f);  // -inf -> +inf
            atomicAdd(&whist[(uint32_t)fminf(fmaxf(tb, 0.0f), 255.0f)], 1u);
        }
        if (k == kRS - 1) {
            lds_wave_fence();  // (the wave's own histogram adds)
            const u4v hc = *reinterpret_cast<const u4v*>(&whist[4 * l]);  // bins 4l..4l+3
            const uint32_t hs = hc.x + hc.y + hc.z + hc.w;
            const uint32_t hi = wscan_u32(hs);
            const uint32_t c0 = hi - hs + hc.x, c1 = c0 + hc.y, c2 = c1 + hc.z, c3 = c2 + hc.w;
            const uint32_t nok = (uint32_t)(c0 <= kRTop) + (uint32_t)(c1 <= kRTop) +
                                 (uint32_t)(c2 <= kRTop) + (uint32_t)(c3 <= kRTop);
            const int bw = (int)wsum_u32(nok) - 1;  // last bin whose cumulative count fits
            thc = (bw < 0 || Kw == 0) ? INFINITY : RwH - (float)(bw + 1) * 0.125f;
            // x_lo = max_w thc_w bounds the complete range, so nothing below
            // the running max of the thresholds published so far is needed
            if (Kw > 0 && l == 0) atomicMax(&sh.kxlo, key32(thc));
            lds_wave_fence();
            thl = fmaxf(thc, unkey32(sh.kxlo));
            // thl in logit units, rounded down: x >= thx whenever x * c >= thl
            thx = thl < INFINITY ? thl / chi - fabsf(thl / chi) * 1.0e-6f - 1.0e-30f : INFINITY;
#pragma unroll
            for (int j = 0; j < kRS; ++j) {
                NIS_RLIST(j, mcs[j] >= thl)
                if (nq - np >= 64u) round(64u);  // (the ring holds at most 127 pending)
            }
        }
        if (k >= kRS) {
            NIS_RLIST(k, m4 >= thx)
            if (nq - np >= 64u) round(64u);
        }
    }
#undef NIS_RLIST

    // ---- stream end ----------------------------------------------------------
    NIS_RTS(2);
    __builtin_amdgcn_s_setprio(0);
    thl = fmaxf(thl, unkey32(sh.kxlo));
    while (nq != np) round(nq - np);  // (at most two rounds)
    mx = wmax_f32(mx);
    z = wsum_f64(z);
    if (l == 0) {
        RRec r;
        r.z = z;
        r.mx = mx;
        r.rw = Rz;
        r.thc = Kw > 0 ? thc : -INFINITY;
        r.nc = nc;
        r.bad = (uint32_t)!(z < INFINITY);
        r.pad = 0u;
        sh.rec[w] = r;
        atomicMax(&sh.kmax, key32(mx));
        if (mx > -INFINITY) atomicMin(&sh.krw, key32(Rz));
        if (nc > 0u) atomicMin(&sh.kth, key32(thc));
        atomicMax(&sh.knc, nc);
        if (!(z < INFINITY)) atomicOr(&sh.kbad, 1u);
    }
    // the row's one draw (sampler.rs:209), by wave 0; the advanced state is
    // stored once the row cannot be declined any more
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
    // ---- B1: every wave's stream, histogram and records are complete ---------
    NIS_RTS(3);
    lds_barrier();
    NIS_RTS(4);
    const bool rv = l < kRW;
    // the row max and R = ceil(M c) (every wave)
    const float M = unkey32(sh.kmax);
    const float R = (M > -INFINITY && fabsf(M * chi) < 1e30f) ? ceilf(M * chi) : 0.0f;
    const int Ri = (int)R;
    if (w == 0) {
        // ---- wave 0: Z, the checks and the cutoff ----------------------------
        const RRec rr = sh.rec[rv ? l : 0];
        const double ZR = r16_sum(rv ? ldexp(rr.z, (int)(rr.rw - R)) : 0.0);
        const double pz = (double)p * ZR * 1099511627776.0;  // p Z in 2^(R - 40) units
        const float xlo = unkey32(sh.kxlo);
        const float rwmin = unkey32(sh.krw), thmin = unkey32(sh.kth);
        const bool fin = (M > -INFINITY) & (M < INFINITY) & (fabsf(M * chi) < 1e6f) & (ZR > 0.0) &
                         (ZR < INFINITY) & (sh.kbad == 0u) & (fmaf(M, chi, -rwmin) <= 100.0f);
        const int bM = fin ? r_bucket(M, chi) : 0;
        const bool xok = (xlo < INFINITY) & (xlo <= M * chi);
        const int blo = xok ? (int)(xlo * (float)kRRes) : 0;  // xlo: a multiple of 1/8
        const int oM = bM >> kRLog, olo = blo >> kRLog;
        RCut cut;
        cut.gp = 0ull;
        cut.pz = pz;
        cut.zr = ZR;
        cut.M = M;
        cut.R = R;
        cut.bp = 0;
        cut.nsel = 0u;
        cut.nab = 0u;
        cut.rej = NIS_REJECT_NONE;
        if (!fin) {
            cut.rej = NIS_REJECT_NONFINITE;
        } else if (sh.knc > (uint32_t)kRC || !(bM - (int)(thmin * (float)kRRes) < kRHB - kRRes)) {
            cut.rej = NIS_REJECT_CAPACITY;
        } else if (!xok) {
            cut.rej = NIS_REJECT_WINDOW;
        } else {
            // level 1: lane l takes octave oM - l; the octaves above olo are
            // complete (their own histogram), octave olo only from blo up (its
            // buckets, summed beside)
            const int o = oM - l;
            const bool oin = l <= oM - olo;
            const bool ofull = l < oM - olo;
            const unsigned long long ovr = ofull ? sh.oct[(uint32_t)o & 31u] : 0ull;
            const int bl = kRRes * olo + l;
            const unsigned long long lv = (bl >= blo && bl <= bM) ? sh.hist[(uint32_t)bl & (kRHB - 1)] : 0ull;
            const unsigned long long omf = r_u40(ovr & 0xFFFFFFFFFFFFull, o, Ri);
            const unsigned long long lm = r_u40(lv & 0xFFFFFFFFFFFFull, olo, Ri);
            const uint32_t onf = (uint32_t)(ovr >> 48), ln = (uint32_t)(lv >> 48);
            const unsigned long long oincl = rscan_u64w(omf);  // the two scans run side by side
            const unsigned long long lincl = rscan_u64w(lm);
            const uint32_t ocincl = wscan_u32(onf), lcincl = wscan_u32(ln);
            const unsigned long long gfull = rbcast_u64(oincl, 63);   // octaves above olo
            const unsigned long long mlo = rbcast_u64(lincl, 63);     // octave olo from blo up
            const uint32_t cfull = bcast_u32(ocincl, 63), clo_n = bcast_u32(lcincl, 63);
            const bool islo = l == oM - olo;
            const unsigned long long om = islo ? mlo : omf;
            const uint32_t on = islo ? clo_n : onf;
            const unsigned long long Go = islo ? gfull : oincl - omf;  // mass of the octaves above
            const uint32_t Co = islo ? cfull : ocincl - onf;
            const unsigned long long gtot = gfull + mlo;  // everything >= blo
            const uint64_t P = __ballot(oin & (on != 0u) & ((double)Go - ldexp(1.0001, o + 1 - Ri + 40) <= pz));
            const uint64_t NEo = __ballot(oin & (on != 0u));
            (void)om;
            // everything below blo is removed: G(blo - 1) - m_up(blo - 1) > p Z
            if (!((double)gtot - r_mup(blo - 1, Ri) > pz) || !P) {
                cut.rej = NIS_REJECT_WINDOW;
            } else {
                const int lp = 63 - __clzll((long long)P);  // deepest passing octave
                const uint64_t up = NEo & ((1ull << lp) - 1ull);
                const int la = up ? 63 - __clzll((long long)up) : -1;  // next non-empty octave above
                // level 2: lane l takes bucket 64 O + 63 - l of O = Op (then Oa)
                int L = -1;
#pragma unroll
                for (int pass2 = 0; pass2 < 2; ++pass2) {
                    if (L < 0 && (pass2 == 0 || la >= 0)) {
                        const int lo2 = pass2 == 0 ? lp : la;
                        const int O = oM - lo2;
                        const unsigned long long GO = rbcast_u64(Go, lo2);
                        const uint32_t CO = bcast_u32(Co, lo2);
                        const int b = kRRes * O + (kRRes - 1) - l;
                        const bool bin = (b >= blo) & (b <= bM);
                        const unsigned long long bv = bin ? sh.hist[(uint32_t)b & (kRHB - 1)] : 0ull;
                        const uint32_t bn = (uint32_t)(bv >> 48);
                        const unsigned long long bm = r_u40(bv & 0xFFFFFFFFFFFFull, O, Ri);
                        const unsigned long long Gb = GO + (rscan_u64w(bm) - bm);
                        const uint32_t Cb = CO + (wscan_u32(bn) - bn);
                        // Op: its deepest passing bucket; Oa (when Op has none):
                        // its lowest non-empty bucket, which then passes
                        const uint64_t sel = pass2 == 0
                                                 ? __ballot((bn != 0u) & ((double)Gb - r_mup(b, Ri) <= pz))
                                                 : __ballot(bn != 0u);
                        if (sel) {
                            L = 63 - __clzll((long long)sel);
                            cut.bp = (int32_t)bcast_u32((uint32_t)b, L);
                            cut.gp = rbcast_u64(Gb, L);
                            cut.nsel = bcast_u32(bn, L);
                            cut.nab = bcast_u32(Cb, L);
                        }
                    }
                }
                // kept masses stay exact integers: b_p within kRDeep octaves of R
                if (L < 0 || (cut.bp >> kRLog) < Ri - kRDeep) cut.rej = NIS_REJECT_WINDOW;
                else if (cut.nsel > (uint32_t)kRMem) cut.rej = NIS_REJECT_BUCKET;
            }
        }
        if (l == 0) sh.cut = cut;
    }
    // every wave: its records, j = 64 i + l (consecutive lanes, consecutive
    // slots), and their masses, while wave 0 searches
    const int nrec = (int)min(nc, (uint32_t)kRC);
    RCand cr[4];
    unsigned long long cmu[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cr[i] = sh.u.s.c.cand[w][64 * i + l];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (64 * i + l >= nrec) cr[i].b = INT32_MIN;  // below any b_p: never kept, never a member
        cmu[i] = r_u40(cr[i].fm, cr[i].b >> kRLog, Ri);
    }
    // ---- B1b: the cutoff bucket is known ------------------------------------
    lds_barrier();
    NIS_RTS(5);
    const RCut cut = sh.cut;
    if (cut.rej != NIS_REJECT_NONE) return cut.rej;
    const int bp = cut.bp;
    // this wave's kept mass above b_p and its members of b_p
    {
        unsigned long long al = 0ull;
        uint32_t mb = 0u;  // bit i: record 64 i + l is a member of b_p
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            al += (cr[i].b > bp) ? cmu[i] : 0ull;
            mb |= (cr[i].b == bp) ? (1u << i) : 0u;
        }
        const unsigned long long at = wsum_u64(al);
        if (__ballot(mb != 0u)) {
            const uint32_t mcnt = (uint32_t)__popc(mb);
            const uint32_t mincl = wscan_u32(mcnt);
            const uint32_t mtot = (uint32_t)__builtin_amdgcn_readlane((int)mincl, 63);
            uint32_t mbase = 0u;
            if (l == 0) mbase = atomicAdd(&sh.nmem, mtot);
            uint32_t slot = bcast_u32(mbase, 0) + mincl - mcnt;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if ((mb >> i) & 1u) {
                    RCand m = cr[i];
                    m.b = w;  // (the owner wave travels in place of the bucket)
                    sh.mem[min(slot, (uint32_t)kRMem - 1)] = m;
                    ++slot;
                }
            }
        }
        if (l == 0) sh.above[w].m = at;
    }
    // ---- B2: members and per-wave sums are complete ------------------------
    lds_barrier();
    NIS_RTS(6);
    const int n = (int)sh.nmem;
    if ((uint32_t)n != cut.nsel) return NIS_REJECT_BUCKET;
    if (w != 0) {
        NIS_RTFLUSH();
        return NIS_REJECT_NONE;
    }
    const unsigned long long gp = cut.gp;
    const double pz = cut.pz;
    // ---- wave 0: rank the members (stable descending order: value, index),
    // pick the wave holding the draw and walk its records -------------------
    if (l < 4) a.rng[4 * (int64_t)row + l] = rst;
    const bool valid = l < n;
    const RCand mr = sh.mem[min(l, kRMem - 1)];
    const unsigned long long Km = valid ? r_key(mr.x, mr.idx) : 0ull;
    const unsigned long long em = valid ? r_u40(mr.fm, bp >> kRLog, Ri) : 0ull;
    unsigned long long pre = 0ull;  // mass of the members ahead of this one
    uint32_t rk = 0u;
    for (int j = 0; j < n; ++j) {
        const unsigned long long Kj = rbcast_u64(Km, j);
        const unsigned long long ej = rbcast_u64(em, j);
        pre += (Kj > Km) ? ej : 0ull;
        rk += (Kj > Km) ? 1u : 0u;
    }
    // sampler.rs:150 in rank order: D = G + pre - e; the kept ones are the
    // longest prefix of ranks with D <= p Z
    const bool pass = valid & ((double)(long long)(gp + pre - em) <= pz);
    uint32_t nkept = (uint32_t)n;
    if (__ballot(valid & !pass)) nkept = wmin_u32((valid && !pass) ? rk : 0xFFFFFFFFu);
    const bool kept = valid & (rk < nkept);
    const uint64_t lastm = __ballot(valid & (rk + 1u == nkept));
    const unsigned long long Kcut = lastm ? rbcast_u64(Km, __ffsll((long long)lastm) - 1) : ~0ull;
    const unsigned long long kmass = kept ? em : 0ull;
    const unsigned long long zk = gp + rbcast_u64(rscan_u64w(kmass), 63);
    // per-wave kept totals: above b_p plus the kept members each wave owns
    const RAbove abv = sh.above[rv ? l : 0];
    unsigned long long T = rv ? abv.m : 0ull;
    for (int j = 0; j < n; ++j) {
        const unsigned long long ej = rbcast_u64(kmass, j);
        const int oj = (int)bcast_u32((uint32_t)mr.b, j);
        T += (l == oj) ? ej : 0ull;
    }
    const unsigned long long Tincl = rscan16_u64(T);
    const double u = sh.u0;
    // the walk stops at the first kept element whose inclusive prefix P
    // reaches r = u Z_kept; P is an integer, so P >= r iff P >= ceil(r)
    const unsigned long long rc = (unsigned long long)ceil(u * (double)zk);
    const uint64_t hw = __ballot(rv & (T > 0ull) & (Tincl >= rc));
    const uint64_t nzw = __ballot(rv & (T > 0ull));
    const int ws = hw ? (__ffsll((long long)hw) - 1) : (63 - __clzll((long long)(nzw | 1ull)));
    unsigned long long acc = rbcast_u64(Tincl - T, ws);
    NIS_RTS(8);
    // the chosen wave's kept records in index order j = 64 i + l (round i,
    // then lane): the round holding the crossing, then the lane
    const int nrw = (int)min(sh.rec[ws].nc, (uint32_t)kRC);
    RCand wr[4];
    unsigned long long me[4], sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[i] = sh.u.s.c.cand[ws][64 * i + l];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool kp = (64 * i + l < nrw) &
                        ((wr[i].b > bp) | ((wr[i].b == bp) & (r_key(wr[i].x, wr[i].idx) >= Kcut)));
        me[i] = kp ? r_u40(wr[i].fm, wr[i].b >> kRLog, Ri) : 0ull;
        sc[i] = rscan_u64w(me[i]);
    }
    int ic = -1, lc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned long long tot = rbcast_u64(sc[i], 63);
        if (ic < 0 && tot > 0ull) {
            if (acc + tot >= rc || i == 3 || 64 * (i + 1) >= nrw) {
                // the crossing (or, if rounding leaves r above every prefix,
                // the last kept record) lies in this round
                const uint64_t hl = __ballot((me[i] > 0ull) & (acc + sc[i] >= rc));
                const uint64_t nzl = __ballot(me[i] > 0ull);
                lc = hl ? (__ffsll((long long)hl) - 1) : (63 - __clzll((long long)nzl));
                ic = i;
            }
            acc += tot;
        }
    }
    if (ic < 0) ic = 0;  // (cannot happen: the chosen wave holds kept mass)
    const uint32_t nab = cut.nab;
    if (l == lc) {
        RCand t = wr[0];
        unsigned long long et = me[0];
#pragma unroll
        for (int i = 1; i < 4; ++i)
            if (i == ic) {
                t = wr[i];
                et = me[i];
            }
        uint32_t tok = t.idx;
        if (u == 0.0) tok = 0u;  // r == 0 stops the reference's walk at index 0
        emit_token(a, row, tok);
        if (a.stats) {
            // 2^(R - M c): units of 2^R -> units of the max element's mass
            const double rho = exp2((double)cut.R - (double)cut.M * c64);
            write_row_stats(a, row, tok, NIS_PATH_DRAW, (double)cut.M / temp,
                            (double)zk / 1099511627776.0 * rho, cut.zr * rho, u,
                            (u == 0.0) ? 0.0 : (double)et / (double)zk, (uint64_t)(nab + nkept), 1);
        }
    }
    NIS_RTS(9);
    NIS_RTFLUSH();
    return NIS_REJECT_NONE;
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
