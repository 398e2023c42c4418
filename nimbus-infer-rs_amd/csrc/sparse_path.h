// sparse_path.h — sparse top-p sampler: one row per 1024-lane workgroup
// (16 wave64s, four per SIMD), for rows whose nucleus holds a small share of
// the vocabulary (V <= 53245, 0 < top_p < 1, T > 0, no top-k; a repetition-
// penalty history is applied by the PEN form, described at sparse_row).
//
// Stream.  Chunk k / lane l of wave w holds float4 slot base_w + 64k + l, so
// each wave owns a contiguous index range of up to 13 chunks.  Every lane
// keeps three nontemporal 16-byte buffer loads in flight ahead of the chunk
// it works on, so each wave's data arrives spread over the whole stream and
// the waves finish together.  As the chunks land each wave adds the masses
// 2^(x c - R_w) to Z in f64 (c = log2(e)/T, R_w an integer reference from
// the wave's first chunk; an element more than 127 octaves above it makes Z
// infinite and the row is declined), keeps its max, and appends every
// float4 holding an element at or above its listing threshold to its LDS
// list (index order, one ballot per chunk).  The threshold thc_w comes from the
// wave's first four chunks: the lower edge of the 1/8-octave bins of x c
// holding at most 44 of their 256 float4 maxima, raised to the running max
// of the thresholds the other waves have published, and at the stream end
// to kSDeep octaves below the largest max seen (nothing deeper is kept).
//
// Cutoff (src/sampler.rs:118-160) without a sort.  The reference keeps
// sorted position pos iff D(pos) = cum_excl(pos) - q(pos) <= p*Z; D is
// non-decreasing in pos, so the kept set is a prefix of the stable order.
// After its stream each wave adds its candidates (the listed elements at or
// above its threshold) to one shared histogram on an absolute grid of 1/64
// octave of x*c (bucket floor(64 * x*c), monotone in x) and to a histogram of
// whole octaves; each bucket holds its count and the exact sum of its
// members' masses in fixed point relative to the bucket's octave.  Every
// element at or above x_lo = max_w thc_w is listed by its wave, so buckets
// from blo = 64 x_lo up are complete.  With G(b) the mass of the buckets
// above b and m_up(b) an upper bound of any mass in b, b_p is the deepest
// non-empty bucket with G(b) - m_up(b) <= p Z:
//   - every bucket below it fails, so its first element and everything after
//     it in sorted order is removed;
//   - every element of the buckets above b_p is kept (the last element y of
//     the next non-empty bucket above has D(y) <= G(b_p) - 2 m(y) < p Z);
//   - the cutoff therefore lies among b_p's members, which are ranked exactly
//     (descending value, ascending index) against sampler.rs:150.
// Elements below blo are removed once G(blo - 1) - m_up(blo - 1) > p Z.
//
// Masses in the tail are integers in units of 2^(R - 40) (R = ceil(M c)),
// held in f64: every sum of them is exact and order-independent, so the
// kept total, the per-wave and per-segment totals and the element walk
// agree to the last bit and the inverse-CDF walk (sampler.rs:209-216)
// always finds its crossing.
//
// Hand-offs after the stream: once every wave's histogram adds are done (one
// barrier), wave 0 finds b_p; a second barrier publishes it; every wave then
// sums its kept mass above b_p per lane segment of its list and lists its
// members of b_p; the last wave to finish that (an LDS counter) ranks the
// members and walks waves -> the chosen wave's list segments -> elements.
// Any step that cannot prove its result returns a reject code before the
// second barrier; the caller then runs the general path on the row.
// The octave histogram keeps 8 copies of each bin (lane & 7 picks one), so
// the 64 lanes of one add round, whose candidates crowd into a few octaves,
// hit up to 8 times as many addresses.
#pragma once
#include "row_common.h"
#include "penalty_bits.h"

namespace nis {

constexpr int kSB = 1024;                   // lanes per workgroup
constexpr int kSW = kSB / 64;               // waves per workgroup
constexpr int kSN = 13;                     // float4 chunks per lane (at most)
constexpr int kSMaxV = kSB * 4 * 13 - 3;    // 53245: 208 chunks of 64 float4 slots
constexpr int kSD = 3;                      // loads in flight per lane ahead of the one in use
constexpr int kSS = 4;                      // sample chunks per wave
constexpr uint32_t kSTop = 44;              // sampled float4 maxima allowed above thc_w
constexpr int kSE = 256;                    // listed float4s per wave
constexpr int kSSeg = kSE / 64;             // list entries per lane segment (at most)
constexpr int kSRes = 64;                   // histogram buckets per octave of x*c
constexpr int kSLog = 6;                    // log2(kSRes)
constexpr int kSHB = 32 * kSRes;            // bucket ring: 32 octaves
constexpr int kSMem = 64;                   // members of the cutoff bucket
constexpr int kSOctC = 8;                   // copies of each octave bin (lane & 7 picks one)
constexpr uint32_t kSNone = 0x80000000u;    // packed bucket of no candidate (below any b_p)
// repetition penalty (sample_rows_sparse_pen_kernel)
constexpr int kSSide = 48;                  // penalised elements per wave
constexpr int kSSlot = 32;                  // float4 slots holding them, per wave
static_assert(kSB == kPB && kSMaxV == kPMaxV, "penalty bitmaps sized for this layout");
constexpr int kSRounds = 4 * kSSeg;         // candidates per lane (at most)
constexpr double kS40 = 1099511627776.0;    // 2^40
// Octaves below the row max past which nothing is kept for top-p < 0.95:
// at most V 2^-22 Z <= 0.013 Z of mass lies there (V <= 53245), and the
// removed mass is at least (1 - p) Z >= 0.05 Z, so every such element is
// removed.  Listing thresholds are never set below (max seen) c - kSDeep.
constexpr float kSDeep = 22.0f;
// TOPK: the k-th largest may lie deeper than that (top-k keeps elements top-p
// alone would remove, at any top-p): 30 octaves, still inside the 32-octave
// histogram ring; a k-th below the listed range declines the row.
constexpr float kSDeepK = 30.0f;

// Optional phase timestamps (profiling builds only; compiled out unless
// NIS_PHASE_TIMING is defined).  Each wave keeps the low 32 bits of the
// 100 MHz clock in registers and writes them out when it leaves: slot
// 256 * row + 8 * wave + i for its own phases, 256 * row + 128 + j for the
// phases of the single-wave steps it ran.
#ifdef NIS_PHASE_TIMING
__device__ unsigned long long nis_sparse_ts[2048 * 256];
#define NIS_TDECL                \
    uint32_t nis_tw_[8] = {};    \
    uint32_t nis_tx_[4] = {};    \
    uint32_t nis_ts_[16] = {};
#define NIS_STS(i) (nis_tw_[i] = (uint32_t)wall_clock64())
#define NIS_STS1(j) (nis_ts_[j] = (uint32_t)wall_clock64())
#define NIS_STX(i) (nis_tx_[i] = (uint32_t)wall_clock64())
#define NIS_TFLUSH()                                                                        \
    do {                                                                                    \
        if (lane_id() == 0 && blockIdx.x < 2048) {                                          \
            unsigned long long* ts_ = &nis_sparse_ts[blockIdx.x * 256];                    \
            _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_) if (nis_tw_[i_])              \
                ts_[8 * wave_id() + i_] = nis_tw_[i_];                                      \
            _Pragma("unroll") for (int j_ = 0; j_ < 16; ++j_) if (nis_ts_[j_])             \
                ts_[128 + j_] = nis_ts_[j_];                                                \
            _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_) if (nis_tx_[i_])              \
                ts_[144 + 4 * wave_id() + i_] = nis_tx_[i_];                                \
        }                                                                                   \
    } while (0)
#else
#define NIS_TDECL
#define NIS_STS(i) \
    do {           \
    } while (0)
#define NIS_STS1(j) \
    do {            \
    } while (0)
#define NIS_STX(i) \
    do {           \
    } while (0)
#define NIS_TFLUSH() \
    do {             \
    } while (0)
#endif

// Stream-end record of one wave (32 bytes, written by its lane 0).
struct alignas(16) SRec {
    double z;     // sum of 2^(x c - R_w) over the wave's elements
    float mx;     // wave max logit
    float rw;     // R_w
    float thc;    // listing threshold in units of x*c (-inf: the wave holds no data)
    uint32_t n;   // float4s listed (may exceed kSE: overflow)
    uint32_t ns;  // penalised elements on the side list (PEN)
    uint32_t pad;
};
// A member of the cutoff bucket.
struct alignas(16) SMem {
    float x;
    uint32_t idx;  // row index
    uint32_t fm;   // octave-relative fixed-point mass
    uint32_t loc;  // owner wave << 16 | lane segment of its entry list
};
// Result of the cutoff search (written by wave 0 between barriers).
struct alignas(16) SCut {
    double gp;        // mass of the buckets above b_p (2^(R-40) units, an integer)
    double pz;        // p * Z (2^(R-40) units; TOPK with split: p * its upper bound)
    double zr;        // Z (units of 2^R)
    double gk;        // TOPK: mass of the buckets above b_k
    int32_t bp;       // b_p
    uint32_t nabove;  // candidates above b_p
    uint32_t reject;
    float M;          // row max logit
    float R;          // ceil(M c)
    int32_t bk;       // TOPK: bucket of the k-th largest
    uint32_t ck;      //   candidates above it
    uint32_t nbk;     //   candidates in it
    uint32_t split;   //   1: its members straddle the k-th (ranked at the walk)
    int32_t bpd;      // deepest bucket the cutoff may lie in (b_p otherwise; TOPK
                      //   with split: [bpd, bp] covers the exact p Z_k)
    uint32_t pad[2];
};

struct WideShared {
    f4v ent[kSW][kSE + 64];        // listed float4s, index order per wave (+ one chunk of slack)
    uint16_t epos[kSW][kSE + 64];  //   their chunk * 64 + lane
    uint32_t whist[kSW][256];      // each wave's sample histogram (1/8-octave bins)
    unsigned long long hist[kSHB]; // [b & (kSHB-1)]: count << 48 | sum of fm, buckets >= blo
    unsigned long long oct[32 * kSOctC]; // the same per octave, kSOctC copies each
    double seg[kSW][64];           // kept mass above b_p per lane segment of the entry lists
    double tw[kSW];                // per-wave kept mass (2^(R-40) units, integers)
    SMem mem[kSMem];               // members of b_p
    SMem kmem[kSMem];              // TOPK: members of b_k (when the k-th largest splits it)
    uint32_t nkmem;
    SRec rec[kSW];
    SCut cut;
    double u0;                     // the draw
    uint32_t nmem;
    uint32_t cnt2;                 // waves done with their kept sums
    // the waves' records reduced as they arrive (order-preserving keys)
    uint32_t kmax;                 // max logit
    uint32_t kxlo;                 // max listing threshold
    uint32_t kthmin;               // min listing threshold of a wave with entries
    uint32_t nmax;                 // largest list
    // repetition penalty only (sparse_row<true>)
    PenBits pb;                        // the history's bitmaps
    f4v sx4[kSW][kSSlot];              // slots met in the stream holding penalised elements
    uint32_t sslot[kSW][kSSlot];       //   slot << 4 | mask of the penalised elements
    double memy[kSMem];                // members' values after the penalty (f64)
    unsigned long long kymax;          // key64 of the largest penalised value (f64)
    uint32_t kmaxp;                    // key32 of the same rounded up to a float
    uint32_t pover;                    // some wave met more than kSSide penalised elements
};
// A penalised element after the stream (16 bytes; kept in its wave's
// sample-histogram slot, which is free by then).
struct alignas(16) SSide {
    double y;      // penalised logit (f64, sampler.rs:94-98)
    uint32_t idx;  // row index
    uint32_t tag;  // bit 0: candidate; after the cutoff: class << 8 | segment << 16
};

// Octave-relative fixed-point mass of a logit with t = x*c already rounded:
// 2^(x c - floor(t)) * 2^24, one rounding in the fma (bounded by 2^25 + eps).
__device__ __forceinline__ uint32_t s_fm(float x, float c, float t) {
    return (uint32_t)(__builtin_amdgcn_exp2f(fmaf(x, c, -floorf(t))) * 16777216.0f);
}
// A sum of fm of octave o in 2^(R - 40) units, as an integer-valued f64:
// exact for o >= R - 16, truncated below.  Sums of these stay below 2^53 and
// are therefore exact and independent of their order.
__device__ __forceinline__ double s_m40(unsigned long long fm, int o, int R) {
    const int sh = o - R + 16;
    const double v = ldexp((double)fm, sh);
    return sh >= 0 ? v : floor(v);
}
// Bucket of t = x*c on the absolute grid: floor(64 t), monotone in x.
__device__ __forceinline__ int s_bucket(float t) {
    int b;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(b) : "v"(t * (float)kSRes));  // floor, then convert
    return b;
}
// Upper bound of the 2^(R - 40)-unit mass of any element in bucket b (its
// upper edge, inflated for the roundings of x*c and exp2).
__device__ __forceinline__ double s_mup(int b, int R) {
    return ldexp((double)__builtin_amdgcn_exp2f((float)((b + 1) & (kSRes - 1)) * (1.0f / kSRes)) *
                     1.0001,
                 ((b + 1) >> kSLog) - R + 40);
}
// Lower bound of the 2^(R - 40)-unit mass of any element in bucket b (its
// lower edge, deflated for the roundings of x*c and exp2 and, more than 16
// octaves below R, for the truncation of s_m40).
__device__ __forceinline__ double s_mdn(int b, int R) {
    const double m = ldexp((double)__builtin_amdgcn_exp2f((float)(b & (kSRes - 1)) * (1.0f / kSRes)) /
                               1.0001,
                           (b >> kSLog) - R + 40);
    return fmax(m - 1.0, 0.0);
}
// Octave-relative fixed-point mass of a penalised element: 2^(yc - floor(t))
// * 2^24 with t = (float)yc, as s_fm is for an f32 logit.
__device__ __forceinline__ uint32_t s_pfm(double yc, float t) {
    return (uint32_t)(__builtin_amdgcn_exp2f((float)(yc - (double)floorf(t))) * 16777216.0f);
}
// max of a float4 and of two floats without the canonicalising moves fmaxf
// adds (NaN inputs are caught through Z later)
__device__ __forceinline__ float s_max4(const f4v& v) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(v.x), "v"(v.y), "v"(v.z));
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(r), "v"(v.w));
    return r;
}
__device__ __forceinline__ float s_max(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// u64 DPP scans (inclusive).  Whole wave, and within each 16-lane row.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned long long dpp0_u64(unsigned long long v) {
    const uint32_t lo = dpp0<CTRL, ROW_MASK>((uint32_t)v), hi = dpp0<CTRL, ROW_MASK>((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wscan_u64(unsigned long long v) {
    v += dpp0_u64<0x111, 0xF>(v);
    v += dpp0_u64<0x112, 0xF>(v);
    v += dpp0_u64<0x114, 0xF>(v);
    v += dpp0_u64<0x118, 0xF>(v);
    v += dpp0_u64<0x142, 0xA>(v);
    v += dpp0_u64<0x143, 0xC>(v);
    return v;
}
__device__ __forceinline__ unsigned long long rscan_u64(unsigned long long v) {
    v += dpp0_u64<0x111, 0xF>(v);
    v += dpp0_u64<0x112, 0xF>(v);
    v += dpp0_u64<0x114, 0xF>(v);
    v += dpp0_u64<0x118, 0xF>(v);
    return v;
}
__device__ __forceinline__ double rscan_f64(double v) {
#define NIS_DPPR(C)                                                                    \
    {                                                                                  \
        const uint64_t b_ = (uint64_t)__double_as_longlong(v);                         \
        const uint64_t lo_ = dpp0<C, 0xF>((uint32_t)b_), hi_ = dpp0<C, 0xF>((uint32_t)(b_ >> 32)); \
        v += __longlong_as_double((long long)((hi_ << 32) | lo_));                     \
    }
    NIS_DPPR(0x111)
    NIS_DPPR(0x112)
    NIS_DPPR(0x114)
    NIS_DPPR(0x118)
#undef NIS_DPPR
    return v;
}
__device__ __forceinline__ uint32_t rscan_u32(uint32_t v) {
    v += dpp0<0x111>(v);
    v += dpp0<0x112>(v);
    v += dpp0<0x114>(v);
    v += dpp0<0x118>(v);
    return v;
}
__device__ __forceinline__ unsigned long long bcast_u64(unsigned long long v, int src) {
    return ((unsigned long long)bcast_u32((uint32_t)(v >> 32), src) << 32) | bcast_u32((uint32_t)v, src);
}
// Reductions over lanes 0..15 (one DPP row), uniform result.
__device__ __forceinline__ float r16_max(float v) {
    v = fmaxf(v, dpp_ninf<0x111>(v));
    v = fmaxf(v, dpp_ninf<0x112>(v));
    v = fmaxf(v, dpp_ninf<0x114>(v));
    v = fmaxf(v, dpp_ninf<0x118>(v));
    return bcast_f32(v, 15);
}
__device__ __forceinline__ double r16_sum(double v) {
#define NIS_DPPD16(C)                                                                  \
    {                                                                                  \
        const uint64_t b_ = (uint64_t)__double_as_longlong(v);                         \
        const uint64_t lo_ = dpp0<C, 0xF>((uint32_t)b_), hi_ = dpp0<C, 0xF>((uint32_t)(b_ >> 32)); \
        v += __longlong_as_double((long long)((hi_ << 32) | lo_));                     \
    }
    NIS_DPPD16(0x111)
    NIS_DPPD16(0x112)
    NIS_DPPD16(0x114)
    NIS_DPPD16(0x118)
#undef NIS_DPPD16
    return bcast_f64(v, 15);
}
__device__ __forceinline__ uint32_t r16_maxu(uint32_t v) {
    v = max(v, dpp0<0x111>(v));
    v = max(v, dpp0<0x112>(v));
    v = max(v, dpp0<0x114>(v));
    v = max(v, dpp0<0x118>(v));
    return bcast_u32(v, 15);
}

// One 64-bit LDS atomic add by the lanes of `mask` only.
__device__ __forceinline__ void lds_add_u64_m(uint64_t mask, uint32_t a, uint64_t v) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_add_u64 %2, %3\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(v)
        : "memory");
}
// Two 64-bit LDS atomic adds by the lanes of `mask` only.
__device__ __forceinline__ void lds_add2_u64_m(uint64_t mask, uint32_t a, uint32_t b, uint64_t v) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_add_u64 %2, %4\n\t"
        "ds_add_u64 %3, %4\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(b), "v"(v)
        : "memory");
}
// One f64 LDS atomic add by the lanes of `mask` only.
__device__ __forceinline__ void lds_add_f64_m(uint64_t mask, uint32_t a, double v) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_add_f64 %2, %3\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(v)
        : "memory");
}
// Two f64 LDS atomic adds by the lanes of `mask` only.
__device__ __forceinline__ void lds_add2_f64_m(uint64_t mask, uint32_t a, uint32_t b, double v) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_add_f64 %2, %4\n\t"
        "ds_add_f64 %3, %4\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(b), "v"(v)
        : "memory");
}
// One 16-byte LDS store by the lanes of `mask` only.
__device__ __forceinline__ void lds_put_b128_m(uint64_t mask, uint32_t a, u4v v) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_write_b128 %2, %3\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(v)
        : "memory");
}
// Two 4-byte LDS stores by the lanes of `mask` only.
__device__ __forceinline__ void lds_put2_u32_m(uint64_t mask, uint32_t a, uint32_t va, uint32_t b,
                                               uint32_t vb) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_write_b32 %2, %3\n\t"
        "ds_write_b32 %4, %5\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(va), "v"(b), "v"(vb)
        : "memory");
}

// PEN: the row may carry a penalty history (its length is checked inside,
// so no load waits before the stream starts).  TOPK: 0 < top_k < V, and any
// top-p above 0 (at 1 or more, top-p is off and the k largest are kept).
template <bool PEN, bool TOPK = false>
__device__ __forceinline__ bool sparse_eligible(const RowArgs a, int row) {
    static_assert(!(PEN && TOPK), "a penalty history with top-k runs the general path");
    if (a.V < 256 || a.V > kSMaxV) return false;
    if (!(a.temperature > 0.0f) || !(a.top_p > 0.0f)) return false;
    if (TOPK) {
        if (!(a.top_k > 0 && a.top_k < (uint64_t)a.V)) return false;
    } else {
        if (!(a.top_p < 1.0f) || (a.top_k > 0 && a.top_k < (uint64_t)a.V)) return false;
    }
    if (PEN) return true;
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1) && g1 > g0) return false;
    return true;
}

// Returns NIS_REJECT_NONE when the row is done, else (uniformly across the
// workgroup) why it must be recomputed; nothing has been written then.
//
// PEN: the row's penalty history is applied on the fly.  Its ids go into two
// LDS bitmaps (elements, and float4 slots) before the stream; a chunk whose
// slots hold none costs one scalar test, and in one that does the owner lanes
// move each penalised logit to their wave's side list and leave -inf in its
// place, so every register-side step skips it.  At the stream end each wave
// takes its side list in f64 (sampler.rs:94-98): the masses join Z, the
// values the max (rounded up), and the ones at or above the listing threshold
// the histograms, with the bucket of (float)(y c) (monotone in y, and equal
// to the f32 bucket rule on unpenalised values).  After the cutoff they join
// the segment sums, the members (ranked on f64 keys) and the final walk,
// placed by row index.
//
// TOPK (top_k_filter, sampler.rs:103-116, then top-p on what it keeps): once
// the histograms are complete every wave finds the bucket b_k holding the
// k-th largest element by counting down from the top (the buckets are
// monotone in x, so the k largest are the buckets above b_k and the largest
// members of b_k).  When b_k's members straddle the k-th (two or more of
// them, more than k in b_k and above), they are listed and ranked, and the
// k-th largest value decides: members at or above it are kept (ties with it
// included), the rest removed.  The top-p cutoff is then searched with
// p Z_k, Z_k the mass kept by top-k, and never below b_k.
template <bool PEN, bool TOPK = false>
__device__ __forceinline__ uint32_t sparse_row(const RowArgs a, const int row, WideShared& sh) {
    const int l = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int V = (int)a.V;
    const gfp rowp = (gfp)(a.logits + (int64_t)row * a.ld);
    const int mis = (int)(((uintptr_t)rowp >> 2) & 3);  // elements before the row in its 16 B block
    const gf4p base = (gf4p)(rowp - mis);
    const int f_lo = mis ? 1 : 0;          // first float4 slot lying fully inside the row
    const int f_hi = (V + mis - 4) >> 2;   // last one
    const int nsl = (V + mis + 3) >> 2;    // slots touching the row
    // wave w owns slots [wbase, wbase + 64 Kw): the same number of chunks
    // for every wave but the last ones
    const int cpw = (((nsl + 63) >> 6) + kSW - 1) / kSW;  // chunks per wave
    const int wbase = 64 * cpw * w;
    const int Kw = min(max((nsl - wbase + 63) >> 6, 0), cpw);
    const int slot0 = wbase + l;
    NIS_TDECL
    NIS_STS(0);

    // the (at most 3 + 3) elements of partial head / tail slots, by one
    // vector load (lane i < 3: element i, lane 3 + i: element V - 6 + 3 + i)
    const float hv = rowp[(l < 3) ? l : ((l < 6) ? V - 6 + l : 0)];
    __builtin_amdgcn_sched_barrier(0);
    // buffer descriptor over the whole slots [0, f_hi]; the partial head slot
    // is redirected to f_lo, slots past f_hi read zeros (both fixed below)
    const uint64_t bptr = (uint64_t)(uintptr_t)base;
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    f4v xv[kSN];
    // Chunk 0 first; then the LDS state every wave shares (its histogram
    // slice and the counters) is cleared and one barrier orders that before
    // any use.  The barrier sits before the other loads: a barrier after a
    // wave's whole batch of loads would wait until the CU has issued them
    // all, which it does only as the row's data arrives.
    xv[0] = nis_buffer_load_f4(rsrc, (Kw > 0) ? 16 * max(slot0, f_lo) : 0x7FFFFFF0, 0, 2);
    __builtin_amdgcn_sched_barrier(0);
    // PEN: the raw history ids (behind chunk 0), and the bitmaps cleared
    const int tid = (int)threadIdx.x;
    uint32_t hid[kPHist / kPB];
    // (too long a history declines the row; the flag is stored once the
    // first barrier is behind, so that no wave waits for the history's
    // length before the row's next loads go out)
    bool hlong = false;
    if constexpr (PEN) {
        hlong = pen_load_ids(a, row, tid, hid);
        pen_clear(sh.pb, tid);
    }
    *reinterpret_cast<u4v*>(&sh.hist[w * (kSHB / kSW) + 2 * l]) = u4v{0u, 0u, 0u, 0u};
    if (l < 32 * kSOctC / kSW) sh.oct[w * (32 * kSOctC / kSW) + l] = 0ull;
    if (w == 0 && l == 0) {
        sh.nmem = 0u;
        sh.nkmem = 0u;
        sh.cnt2 = 0u;
        sh.kmax = 0u;
        sh.kxlo = 0u;
        sh.kthmin = 0xFFFFFFFFu;
        sh.nmax = 0u;
        if (PEN) {
            sh.kymax = 0ull;
            sh.pover = 0u;
            sh.kmaxp = 0u;
        }
    }
    lds_barrier();
    const int voff = 16 * slot0;  // (chunks past the first never hold slot 0)
#define NIS_SLOAD(k)                                                                          \
    do {                                                                                      \
        xv[k] = nis_buffer_load_f4(rsrc, ((k) < Kw) ? voff + 1024 * (k) : 0x7FFFFFF0, 0, 2);  \
    } while (0)
#pragma unroll
    for (int k = 1; k < kSD && k < kSN; ++k) {
        NIS_SLOAD(k);
        __builtin_amdgcn_sched_barrier(0);  // chunk order = issue order
    }
    // the row's RNG state (sampler.rs:209 draws from it once), wave 0 only
    typedef const __attribute__((address_space(1))) uint64_t* gu64p;
    uint64_t rsv = 0;
    if (w == 0) rsv = ((gu64p)(a.rng + 4 * (int64_t)row))[l & 3];
    // PEN: the bitmaps, then bit k of pany: chunk k of this wave has a slot
    // holding a penalised element, and bits 4k..4k+3 of pnl: which elements
    // of this lane's slot in chunk k are penalised
    uint32_t pany = 0u;
    uint64_t pnl = 0ull;
    if constexpr (PEN) {
        pen_set_bits(sh.pb, hid, V, mis);
        if (tid == 0 && hlong) atomicOr(&sh.pover, 1u);
        lds_barrier();
        pen_masks<kSN>(sh.pb, wbase, Kw, l, pany, pnl);
    }

    // The CU serves the waves' loads in wave order, so later waves get their
    // data later and sit on the critical path: they run at a higher priority
    // than the waves ahead of them (dropped to 0 at each wave's stream end).
    __builtin_amdgcn_s_setprio(0);
    if (w >= kSW / 4) __builtin_amdgcn_s_setprio(1);
    if (w >= kSW / 2) __builtin_amdgcn_s_setprio(2);
    if (w >= 3 * kSW / 4) __builtin_amdgcn_s_setprio(3);
    // each wave's sample histogram is its own
    uint32_t* const whist = &sh.whist[w][0];
    *reinterpret_cast<u4v*>(&whist[4 * l]) = u4v{0u, 0u, 0u, 0u};

    const bool edge_wave = (wbase < f_lo) || (wbase + 64 * Kw - 1 > f_hi);
    // (used only by edge waves; the broadcasts wait for the first load only)
    const float h0 = bcast_f32(hv, 0), h1 = bcast_f32(hv, 1), h2 = bcast_f32(hv, 2);
    const float t0 = bcast_f32(hv, 3), t1 = bcast_f32(hv, 4), t2 = bcast_f32(hv, 5);
#define NIS_SFIX(k)                                                                           \
    do {                                                                                      \
        const int fb0 = wbase + (k) * 64;                                                     \
        if (fb0 < f_lo || fb0 + 63 > f_hi)                                                    \
            xv[k] = fix_slot(xv[k], slot0 + (k) * 64, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2); \
    } while (0)

    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const float c = (float)(1.4426950408889634 / temp);     // log2(e) / T
    const float p = a.top_p;
    const f4v ninf4 = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    // PEN: the slots of chunk k holding penalised elements go to the wave's
    // side list whole (with their element mask); -inf stays in their place
    uint32_t ns = 0u;  // this wave's listed slots so far
#define NIS_SPEN(k)                                                                             \
    if constexpr (PEN) {                                                                        \
        if ((pany >> (k)) & 1u) {                                                              \
            const uint32_t s_ = (uint32_t)(slot0 + 64 * (k));                                   \
            const uint32_t nb_ = (uint32_t)(pnl >> (4 * (k))) & 15u;                            \
            const uint64_t mq_ = __ballot(nb_ != 0u);                                           \
            const uint32_t p_ = ns + lane_rank(mq_);                                            \
            if (nb_ != 0u && p_ < (uint32_t)kSSlot) {                                           \
                sh.sx4[w][p_] = xv[k];                                                          \
                sh.sslot[w][p_] = (s_ << 4) | nb_;                                              \
            }                                                                                   \
            ns += (uint32_t)__popcll(mq_);                                                      \
            xv[k] = f4v{(nb_ & 1u) ? -INFINITY : xv[k].x, (nb_ & 2u) ? -INFINITY : xv[k].y,     \
                        (nb_ & 4u) ? -INFINITY : xv[k].z, (nb_ & 8u) ? -INFINITY : xv[k].w};    \
        }                                                                                       \
    }

    // wave reference from the first chunk
    if (Kw == 0) xv[0] = ninf4;
    else if (edge_wave) NIS_SFIX(0);
    NIS_SPEN(0)
    const float m0 = wmax_f32(max4(xv[0]));
    const float Rw = (m0 > -INFINITY && fabsf(m0 * c) < 1e30f) ? ceilf(m0 * c) : 0.0f;
    const float RwH = Rw + 8.0f;  // top of the sample histogram (8 octaves of head room)
    NIS_STS(5);

    // ---- stream: masses, Z, max, listing --------------------------------
    // cz / Rz are opaque copies of c / Rw, so the masses are not merged with
    // identical expressions elsewhere and kept live.
    double z = 0.0;
    float mx = -INFINITY;
    float cz = c, Rz = Rw;
    asm volatile("" : "+v"(cz), "+v"(Rz));
    const uint32_t ent0 = lds_addr(&sh.ent[w][0]), pos0 = lds_addr(&sh.epos[w][0]);
    float thc = INFINITY;  // this wave's sample threshold (x*c units, a multiple of 1/8)
    float thl = INFINITY;  // its listing threshold: thc raised to the waves' running max
    float thx = INFINITY;  // the same in logit units, rounded down
    uint32_t nw = 0;
    float mcs[kSS];
    // (a chunk's entries go from slot min(nw, kSE) on: at most 64 of them land
    // in the list's slack, and a list past kSE entries declines the row)
#define NIS_SLIST(k, cond)                                                                  \
    {                                                                                       \
        const uint64_t mk = __ballot(cond);                                                 \
        const uint32_t slot = __builtin_amdgcn_mbcnt_hi(                                    \
            (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, min(nw, (uint32_t)kSE))); \
        lds_put_x4_u16(mk, ent0 + 16 * slot, xv[k], pos0 + 2 * slot, (uint32_t)((k) * 64 + l)); \
        nw += (uint32_t)__popcll(mk);                                                       \
    }
#define NIS_SSTREAM(FIX)                                                                     \
    _Pragma("unroll") for (int k = 0; k < kSN; ++k) {                                        \
        if (k + kSD < kSN) NIS_SLOAD(k + kSD);                                               \
        __builtin_amdgcn_sched_barrier(0);                                                   \
        if (k >= Kw && k >= kSS) continue;                                                   \
        if (k > 0) {                                                                         \
            if (k >= Kw) xv[k] = ninf4;                                                      \
            else if (FIX) NIS_SFIX(k);                                                       \
            NIS_SPEN(k)                                                                      \
        }                                                                                    \
        const f4v x = xv[k];                                                                 \
        const float e0 = __builtin_amdgcn_exp2f(fmaf(x.x, cz, -Rz));                         \
        const float e1 = __builtin_amdgcn_exp2f(fmaf(x.y, cz, -Rz));                         \
        const float e2 = __builtin_amdgcn_exp2f(fmaf(x.z, cz, -Rz));                         \
        const float e3 = __builtin_amdgcn_exp2f(fmaf(x.w, cz, -Rz));                         \
        z += (double)((e0 + e1) + (e2 + e3));                                                \
        const float m4 = s_max4(x);                                                          \
        mx = s_max(mx, m4);                                                                  \
        if (k < kSS) {                                                                       \
            const float mc = m4 * c;                                                         \
            mcs[k] = mc;                                                                     \
            const float tb = floorf((RwH - mc) * 8.0f); /* -inf -> +inf */                   \
            atomicAdd(&whist[(uint32_t)fminf(fmaxf(tb, 0.0f), 255.0f)], 1u);                 \
        }                                                                                    \
        if (k == kSS - 1) {                                                                  \
            lds_wave_fence();                                                                \
            const u4v hc = *reinterpret_cast<const u4v*>(&whist[4 * l]); /* bins 4l.. */     \
            const uint32_t hs = hc.x + hc.y + hc.z + hc.w;                                   \
            const uint32_t hi = wscan_u32(hs);                                               \
            const uint32_t c0 = hi - hs + hc.x, c1 = c0 + hc.y, c2 = c1 + hc.z, c3 = c2 + hc.w; \
            const uint32_t nok = (uint32_t)(c0 <= kSTop) + (uint32_t)(c1 <= kSTop) +         \
                                 (uint32_t)(c2 <= kSTop) + (uint32_t)(c3 <= kSTop);          \
            const int bw = (int)wsum_u32(nok) - 1; /* last bin whose cumulative count fits */ \
            thc = (bw < 0 || Kw == 0) ? INFINITY : RwH - (float)(bw + 1) * 0.125f;           \
            /* x_lo = max_w thc_w bounds the complete range, so nothing below the */         \
            /* running max of the thresholds published so far is ever needed; the */         \
            /* sample's max goes out too (the depth clamp at the stream end) */             \
            {                                                                                \
                const float msw = wmax_f32(mx);                                              \
                if (l == 0) {                                                                \
                    if (Kw > 0) atomicMax(&sh.kxlo, key32(thc));                             \
                    atomicMax(&sh.kmax, key32(msw));                                         \
                }                                                                            \
            }                                                                                \
            lds_wave_fence();                                                                \
            thl = fmaxf(thc, unkey32(sh.kxlo));                                              \
            /* thl in logit units, rounded down: x >= thx whenever x * c >= thl */           \
            thx = thl < INFINITY ? thl / c - fabsf(thl / c) * 1.0e-6f - 1.0e-30f : INFINITY; \
            _Pragma("unroll") for (int j = 0; j < kSS; ++j) NIS_SLIST(j, mcs[j] >= thl)      \
            NIS_STS(6);                                                                      \
        }                                                                                    \
        if (k >= kSS) NIS_SLIST(k, m4 >= thx)                                                \
    }
    if (edge_wave) {
        NIS_SSTREAM(true)
    } else {
        NIS_SSTREAM(false)
    }
    // A wave whose sample missed the bulk of its data (a masked stretch over
    // its first chunks) sets its threshold too deep and overflows its list.
    // If a higher threshold has been published meanwhile, it lists again
    // from its registers at that one: still every element at or above the
    // final x_lo, which is at least the threshold published now.
    if (nw > (uint32_t)kSE) {  // (wave-uniform)
        const float tpub = unkey32(sh.kxlo);
        if (tpub > thl && tpub < INFINITY) {
            thl = tpub;
            thx = thl / c - fabsf(thl / c) * 1.0e-6f - 1.0e-30f;
            nw = 0u;
#pragma unroll
            for (int k = 0; k < kSN; ++k)
                if (k < Kw) NIS_SLIST(k, max4(xv[k]) >= thx)
        }
    }
#undef NIS_SSTREAM
#undef NIS_SLIST
#undef NIS_SLOAD
#undef NIS_SFIX
#undef NIS_SPEN

    // ---- stream end: this wave's candidates into the histograms ----------
    NIS_STS(1);
    __builtin_amdgcn_s_setprio(0);
    thl = fmaxf(thl, unkey32(sh.kxlo));
    mx = wmax_f32(mx);
    {
        // nothing more than kSDeep octaves below the row max is kept (top-p
        // < 0.95; TOPK: kSDeepK, and rows needing more are declined by the
        // count search): the threshold rises to that depth below the largest
        // max seen (this wave's, or one published), on the 1/8-octave grid,
        // and the raised threshold is published (x_lo, the complete range,
        // follows it)
        const float mref = fmaxf(mx, unkey32(sh.kmax));
        const float tcl = ceilf((mref * c - (TOPK ? kSDeepK : kSDeep)) * 8.0f) * 0.125f;
        if (tcl > thl && tcl < INFINITY) thl = tcl;
        if (l == 0 && Kw > 0 && thl < INFINITY) atomicMax(&sh.kxlo, key32(thl));
    }
    // ---- PEN: this wave's penalised elements, in f64 ------------------------
    // One per lane (row order): the f64 value (sampler.rs:94-98) and its mass
    // into this lane's part of Z; its exact value and its f32 value rounded up
    // into the row maxima (the latter bounds every element's x c); at or above
    // thl, into the histograms.  The records stay for the tail.
    uint32_t nsc = 0u;  // of them at or above the listing threshold (candidates)
    uint32_t nsw = 0u;  // of them on the side list
    if constexpr (PEN) {
        if (ns != 0u) {  // (wave-uniform: most waves meet no penalised element)
            lds_wave_fence();
            const uint32_t nsl = min(ns, (uint32_t)kSSlot);
            const f4v e4 = sh.sx4[w][min(l, kSSlot - 1)];
            const uint32_t sm = (l < (int)nsl) ? sh.sslot[w][min(l, kSSlot - 1)] : 0u;
            const uint32_t cnt = (uint32_t)__popc(sm & 15u);
            const uint32_t incl = wscan_u32(cnt);
            const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            if ((ns > (uint32_t)kSSlot || tot > (uint32_t)kSSide) && l == 0) sh.pover = 1u;
            nsw = min(tot, (uint32_t)kSSide);
            SSide* const srec = reinterpret_cast<SSide*>(&sh.whist[w][0]);
            uint32_t pos = incl - cnt;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (((sm >> q) & 1u) && pos < (uint32_t)kSSide) {
                    uint32_t* const r32 = reinterpret_cast<uint32_t*>(&srec[pos]);
                    r32[0] = __float_as_uint(e4[q]);  // the logit, until the lane below takes it
                    r32[2] = 4u * (sm >> 4) + (uint32_t)q - (uint32_t)mis;
                }
                pos += (sm >> q) & 1u;
            }
            lds_wave_fence();
            const bool sv = l < (int)nsw;
            const u4v rr = *reinterpret_cast<const u4v*>(&srec[min(l, kSSide - 1)]);
            const double y = sv ? pen_value(__uint_as_float(rr.x), (double)a.penalty) : -INFINITY;
            const double yc = y * (double)c;
            const float ts = (float)yc;
            if (sv) {
                z += pen_mass(yc, Rz);
                if (y > -INFINITY) {
                    atomicMax(&sh.kymax, key64(y));
                    atomicMax(&sh.kmaxp, key32(pen_f32_up(y)));
                }
            }
            const bool cand = sv && ts >= thl;
            const uint64_t cmk = __ballot(cand);
            if (cmk) {
                const int b = s_bucket(ts);
                lds_add2_u64_m(cmk, lds_addr(&sh.hist[0]) + 8 * ((uint32_t)b & (uint32_t)(kSHB - 1)),
                               lds_addr(&sh.oct[0]) + 8 * kSOctC * ((uint32_t)(b >> kSLog) & 31u) +
                                   8 * ((uint32_t)l & (kSOctC - 1)),
                               (1ull << 48) | (uint64_t)s_pfm(yc, ts));
            }
            nsc = (uint32_t)__popcll(cmk);
            if (sv) srec[l] = SSide{y, rr.z, cand ? 1u : 0u};
        }
    }
    z = wsum_f64(z);  // (mx was reduced over the wave above)
    NIS_STS(4);
    // the wave's record, its keys and (wave 0) the row's draw go out before
    // its histogram rounds, so that they overlap them
    {
        const uint64_t zb = (uint64_t)__double_as_longlong(z);
        const uint32_t ra = lds_addr(&sh.rec[w]);
        lds_put_b128_m(1ull, ra, u4v{(uint32_t)zb, (uint32_t)(zb >> 32), __float_as_uint(mx),
                                     __float_as_uint(Rz)});
        lds_put_b128_m(1ull, ra + 16, u4v{__float_as_uint(Kw > 0 ? thc : -INFINITY), nw, nsw, 0u});
    }
    // the row's one draw (sampler.rs:209), made by wave 0 off the critical
    // path; wave 0 stores the advanced state once the row cannot be declined
    uint64_t rst = 0;  // wave 0, lane j < 4: word j of the advanced state
    if (w == 0) {
        uint64_t st[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            st[j] = ((uint64_t)bcast_u32((uint32_t)(rsv >> 32), j) << 32) | bcast_u32((uint32_t)rsv, j);
        const double u0 = rng_next_f64(st);
        if (l == 0) sh.u0 = u0;
        rst = (l == 0) ? st[0] : (l == 1) ? st[1] : (l == 2) ? st[2] : st[3];
    }
    if (l == 0) {
        // (the lowest candidate of this wave is at or above its final thl)
        const float thr = Kw > 0 ? thl : -INFINITY;
        atomicMax(&sh.kmax, key32(mx));
        if (nw > 0u || nsc > 0u) atomicMin(&sh.kthmin, key32(thr));
        atomicMax(&sh.nmax, nw);
    }
    // every element of the wave's entries at or above thl (raised to the
    // thresholds published meanwhile) is a candidate; lane l holds entries
    // [l sg, l sg + sg).  The candidates join the shared histograms (bucket:
    // count << 48 | fm, and octave) one candidate per lane per round (a lane
    // holds few of them), the round's element read back from the list by its
    // LDS address.  Each round's bucket (with the element's place) and fm
    // stay in registers for the kept sums after the search.
    const uint32_t ne = min(nw, (uint32_t)kSE);
    const int sg = (int)((ne + 63u) >> 6);
    const int e0 = l * sg;  // the lane's first entry
    uint32_t cm = 0u;       // bit 4 i + q: element q of entry e0 + i is a candidate
#pragma unroll
    for (int i = 0; i < kSSeg; ++i) {
        if (i < sg) {
            const int j = e0 + i;
            f4v v = sh.ent[w][min(j, kSE - 1)];
            if (j >= (int)ne) v = ninf4;
#pragma unroll
            for (int q = 0; q < 4; ++q) cm |= (elem(v, q) * c >= thl) ? (1u << (4 * i + q)) : 0u;
        }
    }
    uint32_t cbk[kSRounds];  // bucket << 4 | (4 i + q); kSNone: no candidate
    uint32_t cfm[kSRounds];  // its fm
    int nrd = 0;             // rounds (wave-uniform)
    {
        const uint32_t hist0 = lds_addr(&sh.hist[0]);
        const uint32_t oct0 = lds_addr(&sh.oct[0]) + 8 * ((uint32_t)l & (kSOctC - 1));
        const float* const el = reinterpret_cast<const float*>(&sh.ent[w][0]) + 4 * e0;
#pragma unroll
        for (int r = 0; r < kSRounds; ++r) {
            cbk[r] = kSNone;
            cfm[r] = 0u;
        }
#pragma unroll
        for (int r = 0; r < kSRounds; ++r) {
            const uint64_t am = __ballot(cm != 0u);
            if (!am) break;
            nrd = r + 1;
            const uint32_t bit = (uint32_t)__builtin_ctz(cm | 0x8000u);  // 15 for no candidate
            const bool has = cm != 0u;
            cm &= cm - 1u;
            const float xq = el[bit];
            const float tq = xq * c;
            const int b = s_bucket(tq);
            const uint32_t fm = s_fm(xq, c, tq);
            lds_add2_u64_m(am, hist0 + 8 * ((uint32_t)b & (uint32_t)(kSHB - 1)),
                           oct0 + 8 * kSOctC * ((uint32_t)(b >> kSLog) & 31u), (1ull << 48) | (uint64_t)fm);
            cbk[r] = has ? (((uint32_t)b << 4) | bit) : kSNone;
            cfm[r] = fm;
        }
    }
    NIS_STS(7);
    NIS_STS(2);

    // ---- B1: every wave's candidates are in the histograms; wave 0 searches
    const int li = min(l, kSW - 1);
    const bool rv = l < kSW;
    lds_barrier();
    // Ring overrun: a wave may have listed candidates more than 31 octaves
    // below the row max (its threshold was clamped against a max that rose
    // later); they alias in the 32-octave ring.  The row max and the lowest
    // candidate bound are final now, so every wave takes the same decision:
    // each subtracts its own such candidates (exact: integer counts and
    // fixed-point masses), and one barrier orders that before the search.
    // Nothing of the complete range is lost: it lies above x_lo >= M c -
    // kSDeepK.  (PEN: the side lists' candidates are not in the rounds, so
    // the search declines such a row instead.)
    bool ringfix = false;
    if constexpr (!PEN) {
        const float Mr = unkey32(sh.kmax);
        const float thr = unkey32(sh.kthmin);
        if ((Mr > -INFINITY) & (Mr < INFINITY) & (fabsf(Mr * c) < 1e6f) & (thr > -INFINITY) &
            (thr < INFINITY)) {
            const int bMr = s_bucket(Mr * c);
            if (!(bMr - (int)(thr * (float)kSRes) < kSHB - kSRes)) {
                const uint32_t hist0 = lds_addr(&sh.hist[0]);
                const uint32_t oct0 = lds_addr(&sh.oct[0]) + 8 * ((uint32_t)l & (kSOctC - 1));
#pragma unroll
                for (int r = 0; r < kSRounds; ++r) {
                    if (r < nrd) {
                        const int b = (int)cbk[r] >> 4;
                        const uint64_t am = __ballot((cbk[r] != kSNone) & (b <= bMr - (kSHB - kSRes)));
                        if (am)
                            lds_add2_u64_m(am, hist0 + 8 * ((uint32_t)b & (uint32_t)(kSHB - 1)),
                                           oct0 + 8 * kSOctC * ((uint32_t)(b >> kSLog) & 31u),
                                           0ull - ((1ull << 48) | (uint64_t)cfm[r]));
                    }
                }
                ringfix = true;
                lds_barrier();
            }
        }
    }
    if (w == 0) {
        NIS_STS(3);
        __builtin_amdgcn_s_setprio(3);
        const u4v ra = *reinterpret_cast<const u4v*>(&sh.rec[li]);
        const float rrw = __uint_as_float(ra.w);
        const double rz = __longlong_as_double((long long)(((uint64_t)ra.y << 32) | ra.x));
        const float M = PEN ? fmaxf(unkey32(sh.kmax), unkey32(sh.kmaxp)) : unkey32(sh.kmax);
        const float R = (M > -INFINITY && fabsf(M * c) < 1e30f) ? ceilf(M * c) : 0.0f;
        const int Ri = (int)R;
        const float xlo = unkey32(sh.kxlo);
        const float thmin = unkey32(sh.kthmin);
        const uint32_t nmax = sh.nmax;
        const bool fin = (M > -INFINITY) & (M < INFINITY) & (fabsf(M * c) < 1e6f);
        const bool xfin = fin & (xlo < INFINITY) & (xlo <= M * c);
        const int blo = xfin ? (int)(xlo * (float)kSRes) : 0;  // xlo: a multiple of 1/8
        const int bM = xfin ? s_bucket(M * c) : 0;
        const int oM = bM >> kSLog, olo = blo >> kSLog;
        // the level-1 reads go out before anything waits on them: octave
        // oM - l for l <= oM - olo, and octave olo's buckets at or above blo
        // (it holds candidates below blo too; its complete part is their sum)
        const int bl = kSRes * olo + l;
        const unsigned long long lv = (bl >= blo && bl <= bM) ? sh.hist[(uint32_t)bl & (kSHB - 1)] : 0ull;
        const int o = oM - l;
        const bool oin = l <= oM - olo;
        unsigned long long ovr = 0ull;
        if (oin && o != olo) {
            const u4v* const oc = reinterpret_cast<const u4v*>(&sh.oct[kSOctC * ((uint32_t)o & 31u)]);
#pragma unroll
            for (int j = 0; j < kSOctC / 2; ++j) {
                const u4v q = oc[j];
                ovr += (((unsigned long long)q.y << 32) | q.x) + (((unsigned long long)q.w << 32) | q.z);
            }
        }
        const double ZR = r16_sum(rv ? ldexp(rz, (int)(rrw - R)) : 0.0);  // exact rescales
        // (TOPK: replaced below by p times the mass top-k keeps, or by its
        // upper bound when b_k's members straddle the k-th; off at p >= 1)
        double pz = (double)p * ZR * kS40;
        NIS_STS1(8);
        SCut cut;
        cut.reject = NIS_REJECT_NONE;
        cut.gp = 0.0;
        cut.pz = pz;
        cut.zr = ZR;
        cut.gk = 0.0;
        cut.bk = 0;
        cut.ck = 0u;
        cut.nbk = 0u;
        cut.split = 0u;
        cut.bpd = 0;
        cut.bp = 0;
        cut.nabove = 0u;
        cut.M = M;
        cut.R = R;
        // (a wave's Z overflows only for an element 127 octaves above its
        // first chunk's max: then ZR is infinite and the row is declined)
        if (!fin || !(ZR > 0.0) || !(ZR < INFINITY)) {
            cut.reject = NIS_REJECT_NONFINITE;
        } else if (!xfin || nmax > (uint32_t)kSE || (PEN && sh.pover != 0u) || oM - olo > 30) {
            cut.reject = NIS_REJECT_CAPACITY;
        } else if (!ringfix && !(bM - (int)(thmin * (float)kSRes) < kSHB - kSRes)) {
            // (PEN) candidates more than 31 octaves below the row max
            cut.reject = NIS_REJECT_CAPACITY;
        } else {
            // level 1.  Octave olo is the deepest lane, so the octaves' prefix
            // sums do not need its complete part, which is summed alongside.
            const uint32_t onr = (uint32_t)(ovr >> 48);
            const double omr = s_m40(ovr & 0xFFFFFFFFFFFFull, o, Ri);
            const double oincl = wscan_f64(omr);
            const double Go = oincl - omr;  // mass of the octaves above
            const uint32_t ocincl = wscan_u32(onr);
            const uint32_t Co = ocincl - onr;
            const unsigned long long lsum = bcast_u64(wscan_u64(lv), 63);
            const double omlo = s_m40(lsum & 0xFFFFFFFFFFFFull, olo, Ri);
            const uint32_t on = (o == olo) ? (uint32_t)(lsum >> 48) : onr;
            const double gtot = bcast_f64(oincl, 63) + omlo;  // everything >= blo
            // ---- TOPK: b_k, the bucket of the k-th largest, by count.  The
            // buckets are monotone in x, so the k largest are the candidates
            // above b_k and the largest of b_k's; all of b_k is kept unless
            // its members straddle the k-th (two or more, more than k in b_k
            // and above), when they are ranked at the walk and only the bounds
            // Z_lo <= Z_k <= Z_hi are known here
            int bk = 0;
            uint32_t ck = 0u, nbk = 0u;
            double gk = 0.0, pzlo = pz;
            bool split = false;
            uint32_t krej = NIS_REJECT_NONE;
            if constexpr (TOPK) {
                const uint64_t K = a.top_k;
                const uint32_t oc = oin ? on : 0u;
                const uint32_t cincl = wscan_u32(oc);
                const uint64_t hit = __ballot(oin & ((uint64_t)cincl >= K));
                if (!hit) {
                    krej = NIS_REJECT_WINDOW;  // the k-th largest lies below the listed range
                } else {
                    const int lk = __ffsll((long long)hit) - 1;
                    const uint32_t CO = bcast_u32(cincl - oc, lk);
                    const double GO = bcast_f64(Go, lk);
                    const int O = oM - lk;
                    // lane l: bucket 64 O + 63 - l (descending)
                    const int b = kSRes * O + (kSRes - 1) - l;
                    const bool bin = (b >= blo) & (b <= bM);
                    const unsigned long long bv = bin ? sh.hist[(uint32_t)b & (kSHB - 1)] : 0ull;
                    const uint32_t bn = (uint32_t)(bv >> 48);
                    const double bm = s_m40(bv & 0xFFFFFFFFFFFFull, O, Ri);
                    const uint32_t bci = wscan_u32(bn);
                    const double bmi = wscan_f64(bm);
                    const uint64_t hb = __ballot((uint64_t)(CO + bci) >= K);
                    if (!hb) {
                        krej = NIS_REJECT_BUCKET;  // octave and bucket counts disagree
                    } else {
                        const int lb = __ffsll((long long)hb) - 1;
                        bk = kSRes * O + (kSRes - 1) - lb;
                        ck = CO + bcast_u32(bci - bn, lb);
                        nbk = bcast_u32(bn, lb);
                        gk = GO + bcast_f64(bmi - bm, lb);
                        split = nbk >= 2u && (uint64_t)ck + nbk > K;
                        // (b_k may lie more than 16 octaves below R: masses
                        // there are truncated to 2^(R-40) units in Z_k, far
                        // below the cutoff's resolution; only the kept range,
                        // b_p and above, must lie within those 16 octaves)
                        const double zhi = gk + bcast_f64(bm, lb);
                        const double zlo = split ? gk + (double)(K - ck) * s_mdn(bk, Ri) : zhi;
                        pz = p >= 1.0f ? (double)INFINITY : (double)p * zhi;
                        pzlo = p >= 1.0f ? (double)INFINITY : (double)p * zlo;
                        cut.zr = p >= 1.0f ? 0.0 : zhi / kS40;
                    }
                }
                cut.pz = pz;
            }
            const uint64_t P = __ballot(oin & (on != 0u) & (Go - ldexp(1.0001, o + 1 - Ri + 40) <= pz));
            const uint64_t NEo = __ballot(oin & (on != 0u));
            // everything below blo is removed: G(blo - 1) - m_up(blo - 1) > p Z
            // (and every sum of kept masses stays an exact f64 integer: below 2^52)
            // (TOPK: everything below b_k >= blo is removed by top-k)
            const bool lo_ok = (TOPK || (gtot - s_mup(blo - 1, Ri) > pz)) & (gtot < 4503599627370496.0);
            if (TOPK && krej != NIS_REJECT_NONE) {
                cut.reject = krej;
            } else if (!P || !lo_ok) {
                cut.reject = NIS_REJECT_WINDOW;
            } else {
                NIS_STS1(9);
                // level 2 for a threshold pzv whose passing octaves are Pm:
                // lane l takes bucket 64 O + 63 - l of O = Op, the deepest
                // passing octave, then (when Op has no passing bucket) of Oa,
                // the next non-empty octave above it.  Returns the lane of the
                // selected bucket (-1: none) and leaves its values on that lane.
                auto level2 = [&](double pzv, uint64_t Pm, int& bs, double& gs, uint32_t& cs,
                                  uint32_t& ns) -> int {
                    const int lp = 63 - __clzll((long long)Pm);  // deepest passing octave
                    const uint64_t up = NEo & ((1ull << lp) - 1ull);
                    const int la = up ? 63 - __clzll((long long)up) : -1;  // next non-empty above
                    int Ls = -1;
#pragma unroll
                    for (int pass2 = 0; pass2 < 2; ++pass2) {
                        if (Ls < 0 && (pass2 == 0 || la >= 0)) {
                            const int lo2 = pass2 == 0 ? lp : la;
                            const int O = oM - lo2;
                            const double GO = bcast_f64(Go, lo2);
                            const uint32_t CO = bcast_u32(Co, lo2);
                            const int b = kSRes * O + (kSRes - 1) - l;
                            const bool bin = (b >= blo) & (b <= bM);
                            const unsigned long long bv = bin ? sh.hist[(uint32_t)b & (kSHB - 1)] : 0ull;
                            const uint32_t bn = (uint32_t)(bv >> 48);
                            const double bm = s_m40(bv & 0xFFFFFFFFFFFFull, O, Ri);
                            const double Gb = GO + (wscan_f64(bm) - bm);
                            const uint32_t Cb = CO + (wscan_u32(bn) - bn);
                            // Op: its deepest passing bucket; Oa (when Op has none):
                            // its lowest non-empty bucket, which then passes
                            const uint64_t sel = pass2 == 0
                                                     ? __ballot((bn != 0u) & (Gb - s_mup(b, Ri) <= pzv))
                                                     : __ballot(bn != 0u);
                            if (sel) {
                                Ls = 63 - __clzll((long long)sel);
                                bs = b;
                                gs = Gb;
                                cs = Cb;
                                ns = bn;
                            }
                        }
                    }
                    return Ls;
                };
                int bsel = 0;
                double gsel = 0.0;
                uint32_t csel = 0, nsel = 0;
                const int L = level2(pz, P, bsel, gsel, csel, nsel);
                // TOPK with b_k split: the same search with p Z_lo finds the
                // shallowest bucket the cutoff may lie in (-1: none)
                int Llo = -1, blsel = 0;
                double glsel = 0.0;
                uint32_t clsel = 0;
                if constexpr (TOPK) {
                    if (split && L >= 0) {
                        const uint64_t Plo =
                            __ballot(oin & (on != 0u) & (Go - ldexp(1.0001, o + 1 - Ri + 40) <= pzlo));
                        uint32_t nlsel = 0;
                        if (Plo) Llo = level2(pzlo, Plo, blsel, glsel, clsel, nlsel);
                    }
                }
                if (L < 0) {
                    cut.reject = NIS_REJECT_WINDOW;
                } else {
                    cut.bp = (int32_t)bcast_u32((uint32_t)bsel, L);
                    cut.gp = bcast_f64(gsel, L);
                    cut.nabove = bcast_u32(csel, L);
                    uint32_t nbp = bcast_u32(nsel, L);
                    cut.bpd = cut.bp;
                    if constexpr (TOPK) {
                        // with b_k split, b_p was found with p Z_hi (the deepest
                        // the cutoff may be); with p Z_lo it may be as shallow
                        // as the deepest bucket passing then.  Every member of
                        // [bpd, bp] is ranked at the walk with the exact p Z_k,
                        // everything above bp is kept, everything below bpd is
                        // removed.  Neither lies below b_k.
                        const int bhi = cut.bp;  // b_p with p Z_hi (exact when not split)
                        const int bdeep = max(bhi, bk);
                        const uint32_t cdeep =  // candidates at or above bdeep
                            bhi >= bk ? bcast_u32(csel + nsel, L) : ck + nbk;
                        int bshal = bdeep;       // the shallow end
                        if (split) {
                            if (Llo < 0) {
                                cut.reject = NIS_REJECT_WINDOW;  // b_lo in another octave: rare
                            } else {
                                bshal = max((int)bcast_u32((uint32_t)blsel, Llo), bk);
                            }
                        }
                        if (bshal == bk) {
                            cut.bp = bk;
                            cut.gp = gk;
                            cut.nabove = ck;
                        } else if (split && Llo >= 0) {
                            cut.bp = bshal;
                            cut.gp = bcast_f64(glsel, Llo);
                            cut.nabove = bcast_u32(clsel, Llo);
                        }  // (else b_p = b_hi, as found)
                        cut.bpd = bdeep;
                        nbp = cdeep - cut.nabove;  // members of [bpd, bp]
                        if (split && nbk > (uint32_t)kSMem) cut.reject = NIS_REJECT_BUCKET;
                        cut.bk = bk;
                        cut.ck = ck;
                        cut.nbk = nbk;
                        cut.gk = gk;
                        cut.split = split ? 1u : 0u;
                    }
                    // the kept range stays within 16 octaves of R (exact fixed point)
                    if ((cut.bpd >> kSLog) < Ri - 16) cut.reject = NIS_REJECT_WINDOW;
                    else if (nbp > (uint32_t)kSMem) cut.reject = NIS_REJECT_BUCKET;
                }
            }
        }
        NIS_STS1(10);
        NIS_STS1(0);
        if (l == 0) sh.cut = cut;
        __builtin_amdgcn_s_setprio(0);
    }
    // ---- B2: the cutoff bucket is known ------------------------------------
    lds_barrier();
    if (w == 0) NIS_STS1(1);
    const SCut cut = sh.cut;
    if (cut.reject != NIS_REJECT_NONE) {
        NIS_TFLUSH();
        return cut.reject;
    }
    NIS_STX(0);
    if (w == 0 && l < 4) a.rng[4 * (int64_t)row + l] = rst;
    const int bp = cut.bp;
    const float M = cut.M, R = cut.R;
    const int Ri = (int)R;
    {
        // this wave's kept mass above b_p per lane segment of its entry list
        // (lane l: entries [l sg, l sg + sg)), and its members of b_p; every
        // element of bucket >= b_p >= blo is listed, and its mass (octave
        // >= R - 16) is an exact integer in 2^(R - 40) units
        // (in 64-bit integers: a kept mass is fm << (octave - R + 16), a shift
        // of 0..16)
        unsigned long long isum = 0ull;
        uint32_t mb = 0u;  // bit 4 i + q: element q of entry i is a member
        // TOPK: b_k split and below the cutoff range: its members are listed
        // too (they fix Z_k); the members of the range [bpd, bp] are listed
        const bool ksplit = TOPK && cut.split != 0u && cut.bk < cut.bpd;
        const int bpd = TOPK ? cut.bpd : bp;
        uint32_t mk = 0u;
#pragma unroll
        for (int r = 0; r < kSRounds; ++r) {
            if (r < nrd) {
                const int b = (int)cbk[r] >> 4;
                const uint32_t fk = (b > bp) ? cfm[r] : 0u;
                isum += (unsigned long long)fk << ((uint32_t)((b >> kSLog) - Ri + 16) & 63u);
                mb |= (b >= bpd && b <= bp) ? (1u << (cbk[r] & 15u)) : 0u;
                if (TOPK) mk |= (ksplit && b == cut.bk) ? (1u << (cbk[r] & 15u)) : 0u;
            }
        }
        if (TOPK && ksplit) {  // (uniform; at most kSMem members, checked above)
            const uint32_t kc = (uint32_t)__popc(mk);
            const uint32_t kincl = wscan_u32(kc);
            const uint32_t ktot = (uint32_t)__builtin_amdgcn_readlane((int)kincl, 63);
            if (ktot) {
                uint32_t base = 0u;
                if (l == 0) base = atomicAdd(&sh.nkmem, ktot);
                uint32_t slot = bcast_u32(base, 0) + kincl - kc;
                while (mk) {
                    const int bit = __ffs(mk) - 1;
                    mk &= mk - 1u;
                    const int e = l * sg + (bit >> 2), q = bit & 3;
                    const float x = reinterpret_cast<const float*>(&sh.ent[w][e])[q];
                    const uint32_t idx = (uint32_t)(4 * (wbase + (int)sh.epos[w][e]) - mis + q);
                    sh.kmem[min(slot, (uint32_t)kSMem - 1)] = SMem{x, idx, s_fm(x, c, x * c), 0u};
                    ++slot;
                }
            }
        }
        if (PEN && nsw != 0u) {
            // the side list: class (1: kept, above b_p; 2: member of b_p), lane
            // segment (the last one whose first entry's slot is at or before
            // the element's slot, so the segments stay in row order) and the
            // kept masses into those segments' sums
            SSide* const srec = reinterpret_cast<SSide*>(&sh.whist[w][0]);
            const bool sv = l < (int)nsw;
            const SSide sd = srec[min(l, kSSide - 1)];
            const double yc = sd.y * (double)c;
            const float ts = (float)yc;
            const int b = s_bucket(ts);
            const bool cand = sv && (sd.tag & 1u) != 0u;
            const uint32_t cls = !cand ? 0u : (b > bp ? 1u : (b == bp ? 2u : 0u));
            const uint32_t fm = s_pfm(yc, ts);
            const unsigned long long km =
                cls == 1u ? (unsigned long long)fm << ((uint32_t)((b >> kSLog) - Ri + 16) & 63u) : 0ull;
            const int jj = l * sg;
            const int fs = (jj < (int)ne) ? (int)sh.epos[w][min(jj, kSE - 1)] : 0x7FFFFFFF;
            uint32_t sseg = 0u;
            uint64_t todo = __ballot(cls != 0u);
            while (todo) {  // (few: the penalised elements at or above b_p)
                const int sl = __ffsll((long long)todo) - 1;
                todo &= todo - 1ull;
                const int ss = (int)bcast_u32((sd.idx + (uint32_t)mis) >> 2, sl) - wbase;
                const uint64_t le = __ballot(fs <= ss);  // a prefix of the segments
                const uint32_t sg_s = le ? (uint32_t)(63 - __clzll((long long)le)) : 0u;
                if (l == sl) sseg = sg_s;
                const unsigned long long ks = bcast_u64(km, sl);
                if (l == (int)sg_s) isum += ks;
            }
            if (sv) srec[l].tag = (sd.tag & 1u) | (cls << 8) | (sseg << 16);
            const uint64_t smk = __ballot(cls == 2u);
            if (smk) {
                uint32_t base = 0u;
                if (l == 0) base = atomicAdd(&sh.nmem, (uint32_t)__popcll(smk));
                const uint32_t slot = bcast_u32(base, 0) + lane_rank(smk);
                if (cls == 2u) {
                    const uint32_t sl = min(slot, (uint32_t)kSMem - 1);
                    sh.mem[sl] = SMem{(float)sd.y, sd.idx, fm, ((uint32_t)w << 16) | sseg};
                    sh.memy[sl] = sd.y;
                }
            }
        }
        const double ssum = (double)isum;
        sh.seg[w][l] = ssum;
        const double tsum = wsum_f64(ssum);
        NIS_STX(1);
        const uint32_t mcnt = (uint32_t)__popc(mb);
        const uint32_t mincl = wscan_u32(mcnt);
        const uint32_t mtot = (uint32_t)__builtin_amdgcn_readlane((int)mincl, 63);
        if (mtot) {
            uint32_t base = 0u;
            if (l == 0) base = atomicAdd(&sh.nmem, mtot);
            uint32_t slot = bcast_u32(base, 0) + mincl - mcnt;
            while (mb) {  // (members are few: at most kSMem per row)
                const int bit = __ffs(mb) - 1;
                mb &= mb - 1u;
                const int e = l * sg + (bit >> 2), q = bit & 3;
                const float x = reinterpret_cast<const float*>(&sh.ent[w][e])[q];
                const uint32_t idx = (uint32_t)(4 * (wbase + (int)sh.epos[w][e]) - mis + q);
                sh.mem[min(slot, (uint32_t)kSMem - 1)] =
                    SMem{x, idx, s_fm(x, c, x * c), ((uint32_t)w << 16) | (uint32_t)l};
                if constexpr (PEN) sh.memy[min(slot, (uint32_t)kSMem - 1)] = (double)x;
                ++slot;
            }
        }
        if (l == 0) sh.tw[w] = tsum;
        NIS_STX(2);
    }
    // ---- the last wave to finish its sums ranks the members and walks -------
    NIS_STS(6);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    uint32_t done2 = 0u;
    if (l == 0) done2 = atomicAdd(&sh.cnt2, 1u);
    done2 = bcast_u32(done2, 0);
    NIS_STX(3);
    if (done2 != (uint32_t)(kSW - 1)) {
        NIS_TFLUSH();
        return NIS_REJECT_NONE;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    NIS_STS1(3);
    __builtin_amdgcn_s_setprio(3);

    double pz = cut.pz;
    const double gp = cut.gp;
    double zrs = cut.zr;
    const int n = (int)min(sh.nmem, (uint32_t)kSMem);
    const u4v mr = *reinterpret_cast<const u4v*>(&sh.mem[min(l, kSMem - 1)]);
    const float xm = __uint_as_float(mr.x);
    const uint32_t im = mr.y;
    // TOPK with b_k split: its members (those of b_p when b_k = b_p) ranked
    // by (value desc, index asc); the k-th largest value keeps every member
    // at or above it, and Z_k, hence p Z_k, is now exact
    uint32_t kthk = 0u;
    if constexpr (TOPK) {
        if (cut.split != 0u) {
            const bool same = cut.bk >= cut.bpd;  // b_k is the deep end of the range
            const int nk = same ? n : (int)min(sh.nkmem, (uint32_t)kSMem);
            const SMem kq = sh.kmem[min(l, kSMem - 1)];
            const float xk = same ? xm : kq.x;
            const uint32_t ik = same ? im : kq.idx;
            const uint32_t fk = same ? mr.z : kq.fm;
            const bool kv = (l < nk) & (!same || s_bucket(xm * c) == cut.bk);
            const unsigned long long Kk = kv ? (((unsigned long long)key32(xk) << 32) | (uint32_t)~ik) : 0ull;
            uint32_t rk = 0u;
            for (int j = 0; j < nk; ++j) rk += (bcast_u64(Kk, j) > Kk) ? 1u : 0u;
            const uint64_t kl = __ballot(kv & ((uint64_t)rk + cut.ck + 1u == a.top_k));
            kthk = key32(bcast_f32(xk, kl ? __ffsll((long long)kl) - 1 : 0));
            const bool live = kv & (key32(xk) >= kthk);
            const double zk_ = cut.gk + wsum_f64(live ? s_m40(fk, (int)floorf(xk * c), Ri) : 0.0);
            pz = p >= 1.0f ? (double)INFINITY : (double)p * zk_;
            zrs = p >= 1.0f ? 0.0 : zk_ / kS40;
        }
    }
    // (TOPK: members below the k-th largest value are removed; kthk is 0
    // unless b_k is split, and members above b_k lie above it)
    const bool valid = (l < n) & (key32(xm) >= kthk);
    double ym = 0.0;  // PEN: the member's value in f64
    if constexpr (PEN) ym = sh.memy[min(l, kSMem - 1)];
    const float tm = PEN ? (float)(ym * (double)c) : xm * c;
    const double em = valid ? s_m40(mr.z, (int)floorf(tm), Ri) : 0.0;
    // stable descending order of sampler.rs:140: value, then index (PEN: the
    // f64 value's key, the index compared on its own)
    const unsigned long long Km =
        !valid ? 0ull : PEN ? key64(ym) : (((unsigned long long)key32(xm) << 32) | (uint32_t)~im);
    NIS_STS1(11);
    double pre = 0.0;
    uint32_t rk = 0u;  // members ahead of this one
#pragma unroll 4
    for (int j = 0; j < n; ++j) {
        const unsigned long long Kj = bcast_u64(Km, j);
        const double ej = bcast_f64(em, j);
        bool ahead = Kj > Km;
        if constexpr (PEN) ahead |= (Kj == Km) & (bcast_u32(im, j) < im);
        pre += ahead ? ej : 0.0;
        rk += ahead ? 1u : 0u;
    }
    NIS_STS1(12);
    const bool kept = valid & (gp + pre - em <= pz);  // sampler.rs:150
    const uint64_t keptm = __ballot(kept);
    const uint32_t nkept = (uint32_t)__popcll(keptm);
    // the last kept member (the smallest key; the kept ones are the nkept
    // largest, the keys being distinct); elements of b_p at or above it are kept
    const uint64_t lastm = __ballot(valid & (rk + 1u == nkept));
    const unsigned long long Kcut = lastm ? bcast_u64(Km, __ffsll((long long)lastm) - 1) : ~0ull;
    const uint32_t Icut = lastm ? bcast_u32(im, __ffsll((long long)lastm) - 1) : 0u;  // (PEN)
    // the kept members join their wave's and their segment's kept mass
    {
        const int mw = min((int)(mr.w >> 16), kSW - 1), ms = (int)(mr.w & 63u);
        lds_add2_f64_m(keptm, lds_addr(&sh.tw[mw]), lds_addr(&sh.seg[mw][ms]), em);
    }
    lds_wave_fence();
    const double T = rv ? sh.tw[li] : 0.0;
    const double Tincl = rscan_f64(T);  // (lanes 0..15 hold the waves)
    const double zk = bcast_f64(Tincl, 15);
    const double u = sh.u0;
    const double r = u * zk;
    const uint64_t hw = __ballot(rv & (T > 0.0) & (Tincl >= r));
    const int ws = hw ? (__ffsll((long long)hw) - 1) : 0;
    const double runw = bcast_f64(Tincl - T, ws);
    NIS_STS1(4);
    // the chosen wave's list segments
    const double Sl = sh.seg[ws][l];
    NIS_STS1(5);
    const double Sincl = wscan_f64(Sl);
    const uint64_t hs = __ballot((Sl > 0.0) & (runw + Sincl >= r));
    const int ls = hs ? (__ffsll((long long)hs) - 1) : 0;
    const double runl = bcast_f64(runw + Sincl - Sl, ls);
    // that segment's elements in index order, one per lane (lane j: element
    // j % 4 of the segment's entry j / 4)
    const uint32_t nes = min(sh.rec[ws].n, (uint32_t)kSE);
    const int sgs = (int)((nes + 63u) >> 6);
    const int je = ls * sgs + (l >> 2);
    const int jec = min(je, kSE - 1);
    const float xe = reinterpret_cast<const float*>(&sh.ent[ws][jec])[l & 3];
    const uint32_t ide = (uint32_t)(4 * (64 * cpw * ws + (int)sh.epos[ws][jec]) - mis + (l & 3));
    const float te = xe * c;
    const int be = s_bucket(te);
    bool kje;
    double ee;
    uint32_t idl = ide;  // the lane's row index
    int le;              // the lane holding the drawn element
    if constexpr (!PEN) {
        const unsigned long long Ke = ((unsigned long long)key32(xe) << 32) | (uint32_t)~ide;
        // (members: the cutoff range [bpd, bp], a single bucket but for TOPK)
        kje = (l < 4 * sgs) & (je < (int)nes) &
              ((be > bp) | ((be >= (TOPK ? cut.bpd : bp)) & (be <= bp) & (Ke >= Kcut)));
        ee = kje ? s_m40(s_fm(xe, c, te), (int)floorf(te), Ri) : 0.0;
        NIS_STS1(6);
        const double pe_incl = rscan_f64(ee);
        const uint64_t he = __ballot(kje & (runl + pe_incl >= r));
        le = he ? (__ffsll((long long)he) - 1) : 0;
    } else {
        // lanes 0..15: the segment's listed elements (row order); lanes 16..63:
        // the chosen wave's side list, the kept ones of this segment taking part
        const bool reg = (l < 4 * sgs) & (je < (int)nes);
        const unsigned long long kd = key64((double)xe);
        const bool ge = (kd > Kcut) | ((kd == Kcut) & (ide <= Icut));
        const bool kreg = reg & ((be > bp) | ((be == bp) & ge));
        const double er = kreg ? s_m40(s_fm(xe, c, te), (int)floorf(te), Ri) : 0.0;
        bool ks = false;  // lane >= 16: a kept side element of this segment
        double es = 0.0;  //   and its mass
        const uint32_t nss = min(sh.rec[ws].ns, (uint32_t)kSSide);
        if (nss != 0u) {
            const SSide* const srec = reinterpret_cast<const SSide*>(&sh.whist[ws][0]);
            const int ts_ = l - 16;
            const bool sl_ = (ts_ >= 0) & (ts_ < (int)nss);
            const SSide sd = srec[min(max(ts_, 0), kSSide - 1)];
            const uint32_t cls = (sd.tag >> 8) & 0xFFu;
            const unsigned long long kds = key64(sd.y);
            ks = sl_ & ((sd.tag >> 16) == (uint32_t)ls) &
                 ((cls == 1u) | ((cls == 2u) & ((kds > Kcut) | ((kds == Kcut) & (sd.idx <= Icut)))));
            const double ycs = sd.y * (double)c;
            const float tss = (float)ycs;
            es = ks ? s_m40(s_pfm(ycs, tss), (int)floorf(tss), Ri) : 0.0;
            if (l >= 16) idl = sd.idx;
        }
        kje = (l < 16) ? kreg : ks;
        ee = (l < 16) ? er : es;
        NIS_STS1(6);
        // inclusive prefix in row order: the listed elements' scan, plus every
        // kept side element below; a side element's own prefix adds the scan
        // of the last listed position below it
        const double pr = rscan_f64(l < 16 ? er : 0.0);
        double pe = (l < 16) ? pr : es;
        const uint64_t regm = __ballot(reg);
        uint64_t svm = __ballot((l >= 16) & ks);
        while (svm) {  // (few: the kept penalised elements of this segment)
            const int sl = __ffsll((long long)svm) - 1;
            svm &= svm - 1ull;
            const double e1 = bcast_f64(es, sl);
            const uint32_t i1 = bcast_u32(idl, sl);
            if (idl > i1) pe += e1;
            const uint64_t below = regm & __ballot(idl < i1);
            const double rp = below ? bcast_f64(pr, 63 - __clzll((long long)below)) : 0.0;
            if (l == sl) pe += rp;
        }
        // the crossing: the lowest row index whose inclusive prefix reaches r
        // (lane order is row order when no side element takes part)
        const bool hit = kje & (runl + pe >= r);
        uint64_t he = __ballot(hit);
        if (he >> 16) {
            uint32_t imin = hit ? idl : 0xFFFFFFFFu;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) imin = min(imin, (uint32_t)__shfl_xor((int)imin, o));
            he = __ballot(hit & (idl == imin));
        }
        le = he ? (__ffsll((long long)he) - 1) : 0;
    }
    if (l == le) {
        const uint32_t tok = (u == 0.0) ? 0u : idl;  // r == 0 stops the reference's walk at index 0
        emit_token(a, row, tok);
        if (a.stats) {
            const double prob = (u == 0.0) ? 0.0 : ee / zk;
            // 2^(R - M c): units of 2^R -> units of the max element's mass
            double Mx = (double)M;
            double rho = (double)__builtin_amdgcn_exp2f(-fmaf(M, c, -R));
            if constexpr (PEN) {  // the exact max after the penalty
                Mx = fmax((double)unkey32(sh.kmax), unkey64(sh.kymax));
                rho = (double)__builtin_amdgcn_exp2f(-(float)(Mx * (double)c - (double)R));
            }
            write_row_stats(a, row, tok, NIS_PATH_DRAW, Mx / temp, zk / kS40 * rho,
                            zrs * rho, u, prob, (uint64_t)(cut.nabove + nkept), 1);
        }
    }
    NIS_STS1(7);
    NIS_TFLUSH();
    return NIS_REJECT_NONE;
}

}  // namespace nis
