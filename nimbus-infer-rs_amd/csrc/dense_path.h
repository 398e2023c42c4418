// dense_path.h — top-p rows whatever the size of their nucleus: one row per
// 1024-lane workgroup (16 wave64s, four per SIMD), the row held in VGPRs
// (V <= 53245), for 0 < top_p < 1, T > 0 and no top-k (src/sampler.rs:118-160,
// 183-216); the PEN form also applies a repetition-penalty history
// (sampler.rs:83-101, described at the end of this comment).
//
// Layout and stream.  Wave w owns a contiguous run of Kw 64-slot chunks of
// the row's float4 slots (the chunks split as evenly as they go over the
// waves), lane l of chunk k holds slot wbase + 64 k + l, and every lane
// keeps kDD loads in flight ahead of the chunk it works on.  As a chunk
// lands each lane computes its four
// masses e = 2^(x c - R_z) (c = log2(e) / T split as c_hi + c_lo, R_z the
// wave's integer reference, raised with its running max so that the masses
// near the max have small arguments) into the wave's f64 total, and adds
// every element to ONE shared histogram:
// bucket j = floor(64 f32(x c_hi)) on an absolute grid (monotone in x; a
// ring of 8192 buckets = 128 octaves), holding count << 48 | the sum of the
// octave-relative fixed-point masses fm = floor(2^(x c - floor(j / 64)) 2^24)
// (derived from e by an exact power-of-two scaling).  Sums of fm are exact
// integers, so the histogram is the same in any order of the adds.  A wave
// folds elements more than 64 octaves below its first reference into that
// floor octave (one bucket per lane, so -inf entries do not all add to one
// address).  A row whose max lies 64 or more octaves above a wave's first
// reference (that wave's unfolded range would alias into the searched
// octaves) has its ring built again from the registers after the stream,
// every floor raised to at least 127 octaves below the row max; a wave's
// first reference above the row's declines the row.  A wave whose first
// chunk holds nothing above -inf takes its first reference from all its
// chunks.
//
// Cutoff without a sort.  The reference keeps sorted position pos iff
// D(pos) = cum_excl(pos) - q(pos) <= p Z (sampler.rs:147-154); D is
// non-decreasing in pos, so the kept set is a prefix of the stable order
// (value descending, index ascending).  With G(b) the mass of the buckets
// above b (2^(R - 44) units, R = ceil(M c)) and m_up(b) an upper bound of one
// element's mass in b, b_p is the deepest non-empty bucket with
// G(b) - m_up(b) <= p Z, found by one block-wide scan over the 64 octaves
// below R (4 buckets per lane).  Every bucket below b_p fails, so its first
// element and everything after it in sorted order is removed; the last
// element y of the next non-empty bucket above b_p has D(y) = G(b_p) - 2 e_y
// <= G(b_p) - m_up(b_p) <= p Z, so every element above b_p is kept.  The
// cutoff lies among b_p's members; when they are more than 64 they are
// histogrammed again at 64 times the resolution (floor(64^2 x c_hi), then
// 64^3), the same argument picking the sub-bucket, until at most 64 remain;
// those are ranked exactly (descending value, ascending index) against
// sampler.rs:150.  A row whose cutoff bucket still holds more than 64
// members at 64^3 buckets per octave (exact ties) is declined.
//
// Kept masses.  kept(x, i) <=> F(x) > B or (F(x) == B and key(x, i) >=
// Kcut), with F the final level's bucket function, B the final bucket and
// Kcut the key of the last kept member.  After the cutoff the row is listed
// once more on whichever side of b_p holds fewer elements: every float4 that
// may hold a kept element (few kept: the rest are removed), or every one
// that may hold a removed element (few removed: the rest are kept).  Those
// float4s are recomputed exactly, compacted one per lane; every other float4
// keeps its stream mass or 0.  A row where neither side fits the lists
// recomputes every float4 in registers instead.  The walk (sampler.rs:209-
// 216) then goes waves -> the chosen wave's chunks -> lanes -> elements over
// those per-float4 kept masses, and the drawn token's probability uses its
// mass computed in f64.
//
// PEN: the history's ids go into LDS bitmaps before the stream (as for the
// sparse kernel), so each wave holds one bit per chunk (pany) and each lane a
// 4-bit mask per chunk of its own slot's penalised elements (pnl).  Every
// register pass skips a penalised element: the stream works on a copy of a
// flagged chunk with -inf in its place, and after the cutoff search each
// lane parks its penalised logits in the (then free) histogram ring and puts
// -inf in their register places.  After each pass, each lane visits its own
// penalised elements one by one (few per lane; each_pen) with y = pen(x) in
// f64: the mass 2^(y c - R_z) from the f64 argument, the bucket
// functions floor(64^L T(y)) with T(v) = (float)(v c_hi) (for an f32 logit
// T(x) = f32(x c_hi), so one monotone function orders plain and penalised
// values alike), the max (y rounded up bounds every bucket, and moves the
// wave's reference when it must; the exact f64 max serves the statistics),
// the members, ranked on (key64(value), index) pairs, and the kept masses,
// added to their float4s' entries.  Every float4 holding a penalised
// element is listed on either side of the cutoff, so the unlisted float4s
// are plain.
//
// Any row this path cannot prove returns a reject code before anything is
// written, and the caller runs the general path on it.
#pragma once
#include "resident_path.h"
#include "sparse_path.h"
#include "penalty_bits.h"

namespace nis {

constexpr int kDB = 1024;                  // lanes per workgroup
constexpr int kDW = kDB / 64;              // waves per workgroup
constexpr int kDN = 13;                    // float4 chunks per lane (at most)
constexpr int kDMaxV = kDB * 4 * kDN - 3;  // 53245
constexpr int kDD = 3;                     // loads in flight per lane ahead of the one in use
constexpr int kDRing = 8192;               // histogram ring: 128 octaves of 64 buckets
constexpr int kDSpan = 64;                 // octaves searched below R
constexpr int kDL = 128;                   // listed float4s per wave (one side of the cutoff)
constexpr int kDMem = 64;                  // members ranked exactly
constexpr int kDLevels = 3;                // bucket resolutions: 64, 64^2, 64^3 per octave
constexpr int kDPenLane = 2 * kDRing / kDB;  // PEN: penalised elements one lane's slots may hold

enum { kDKeptSide = 0, kDRemovedSide = 1, kDBrute = 2 };

// Optional phase timestamps (profiling builds only, compiled out unless
// NIS_DENSE_TIMING is defined): each wave keeps the 100 MHz clock of its
// phases in registers and lane 0 stores them at slot 16 (16 row + wave) + i.
#ifdef NIS_DENSE_TIMING
__device__ unsigned long long nis_dense_ts[2048 * kDW * 16];
#define NIS_DTDECL unsigned long long nis_dt_[16] = {};
#define NIS_DTS(i) (nis_dt_[i] = wall_clock64())
#define NIS_DTFLUSH()                                                                   \
    do {                                                                                \
        if (lane_id() == 0 && blockIdx.x < 2048) {                                      \
            _Pragma("unroll") for (int i_ = 0; i_ < 16; ++i_)                            \
                nis_dense_ts[16 * (kDW * blockIdx.x + wave_id()) + i_] = nis_dt_[i_];    \
        }                                                                               \
    } while (0)
#else
#define NIS_DTDECL
#define NIS_DTS(i) \
    do {           \
    } while (0)
#define NIS_DTFLUSH() \
    do {              \
    } while (0)
#endif

// Stream-end record of one wave (lane 0 writes it).
struct alignas(16) DRec {
    float mx;        // wave max logit
    float rz;        // final reference R_z
    float rw0;       // first reference (the wave folds what lies 64 octaves below it)
    uint32_t flags;  // bit 0: NaN seen; bit 1: the wave holds data
};
// A wave's deepest passing bucket of the cutoff search.
struct alignas(16) DCand {
    unsigned long long g;  // mass of the buckets above it (2^(R - 44) units)
    int32_t j;             // the bucket (INT32_MAX: none)
    uint32_t n;            // its count
    uint32_t nab;          // elements above it
    uint32_t pad;
};
// The cutoff, as the waves need it after the member ranking.
struct alignas(16) DCut {
    unsigned long long kcut;  // key of the last kept member (~0: no member kept)
    unsigned long long g;     // mass above the final bucket
    int32_t bj;               // final bucket (level lv)
    int32_t lv;               // its level
    uint32_t nab;             // elements above it
    uint32_t nkept;           // kept members
    uint32_t nsel;            // its members
    uint32_t rej;
    uint32_t kidx;            // PEN: row index of the last kept member (kcut: key64 of its value)
};
// The listed float4s of one side of the cutoff; PEN reuses the space for the
// history bitmaps, which are read before the stream.
struct DList {
    f4v ent[kDW][kDL];        // listed float4s, per wave
    uint16_t epos[kDW][kDL];  //   chunk * 64 + lane
};

struct NucleusShared {
    unsigned long long ring[kDRing];  // [j & (kDRing - 1)]: count << 48 | sum of fm
    union {
        DList l;                      // one side of the cutoff
        PenBits pb;                   // PEN: the history (set-up only)
    } u;
    RCand mem[kDMem];                 // members of the final bucket (PEN: idx bit 31 = penalised)
    unsigned long long mkey[kDMem];   //   their stable-order keys (ranking; PEN: key64 of the value)
    unsigned long long mmass[kDMem];  //   and masses (2^(R - 44) units)
    uint32_t midx[kDMem];             //   PEN: their row indices
    unsigned long long sub[64];       // refinement histogram of the cutoff bucket
    float walk[kDN][64];              // the chosen wave's per-float4 kept masses
    float em4[kDW][kDN][64];          // each lane's float4 masses (2^R_z units), then
                                      //   kept masses (listed rows, after the cutoff)
    uint32_t kmax;                    // the waves' maxima, reduced as they arrive (key32)
    uint32_t krw0;                    //   their first references (min, key32)
    uint32_t krw0hi;                  //   the highest of those of the waves holding
                                      //   data (max, key32)
    uint32_t fnan;                    //   a NaN seen
    uint32_t kpl;                     // PEN: the plain elements' max (key32; kmax also
                                      //   holds the penalised values rounded up)
    unsigned long long kymax;         // PEN: the penalised values' exact max (key64)
    uint32_t pover;                   // PEN: bit 0: the history is longer than the bitmaps
                                      //   take; bit 1: a lane holds more than kDPenLane
                                      //   penalised elements
    double my[kDMem];                 // PEN: the penalised members' values
    unsigned long long wtm[kDW];      // search: each wave's bucket mass
    uint32_t wtc[kDW];                //   and count
    DCand cand[kDW];
    double tw[kDW];                   // per-wave kept mass (2^R units)
    DCut cut;
    double u0;                        // the draw
    uint32_t nmem;
    uint32_t over;                    // a wave's side list overflowed
};

// PEN: the row may carry a penalty history (its length is checked inside).
template <bool PEN>
__device__ __forceinline__ bool dense_eligible(const RowArgs a, int row) {
    if (a.V < 256 || a.V > kDMaxV) return false;
    if (!(a.temperature > 0.0f) || !(a.top_p > 0.0f) || !(a.top_p < 1.0f)) return false;
    if (a.top_k > 0 && a.top_k < (uint64_t)a.V) return false;
    if (PEN) return true;
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1) && g1 > g0) return false;
    return true;
}

// min of a float4 and max of two floats without canonicalising moves
__device__ __forceinline__ float d_min4(const f4v& v) {
    float r;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(v.x), "v"(v.y), "v"(v.z));
    asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(r), "v"(v.w));
    return r;
}
__device__ __forceinline__ float d_vmax(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// floor to int, saturating (-inf -> INT32_MIN; NaN -> 0, never used)
__device__ __forceinline__ int d_flr(float v) {
    int b;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(b) : "v"(v));
    return b;
}
// A bucket's fm sum (low 48 bits of v) in octave o as an integer in
// 2^(R - 44) units: exact for o >= R - 20, truncated below (every element's
// mass is at most 2^(R - o + ...) <= 2^44 units, so totals stay below 2^61).
__device__ __forceinline__ unsigned long long d_u44(unsigned long long v, int o, int R) {
    const int d = R - o;
    const unsigned long long f = (v & 0xFFFFFFFFFFFFull) << 20;
    return d <= 0 ? f : (d < 64 ? (f >> (uint32_t)d) : 0ull);
}
// Upper bound of one element's mass in level-lv bucket F (64^(lv+1) buckets
// per octave): its upper edge, inflated for the roundings of x c and exp2;
// 2^(R - 44) units.
__device__ __forceinline__ double d_mup(int F, int lv, int R) {
    const int sh = 6 * (lv + 1);
    const int Fp = F + 1;
    const float fr = (float)(Fp & ((1 << sh) - 1)) * __builtin_amdgcn_ldexpf(1.0f, -sh);
    return ldexp((double)__builtin_amdgcn_exp2f(fr) * 1.0001, (Fp >> sh) - R + 44);
}
// Kept test of element (x, idx) against the cutoff (F at resolution chiL).
__device__ __forceinline__ bool d_kept(float x, uint32_t idx, float chiL, int B,
                                       unsigned long long kcut) {
    const int F = d_flr(x * chiL);
    return (F > B) | ((F == B) & (r_key(x, idx) >= kcut));
}
// PEN: a float4 with its penalised elements (bits of nb) set to -inf
__device__ __forceinline__ f4v d_mask4(const f4v& x, uint32_t nb) {
    return f4v{(nb & 1u) ? -INFINITY : x.x, (nb & 2u) ? -INFINITY : x.y, (nb & 4u) ? -INFINITY : x.z,
               (nb & 8u) ? -INFINITY : x.w};
}
// T(y) = (float)(y c_hi) of a penalised value: the f32 rounding of its f64
// product, as f32(x c_hi) is for a logit (whose product is exact in f64).
__device__ __forceinline__ float d_pt(double y, double chid) { return (float)(y * chid); }
// Octave-relative fixed-point mass of a penalised value in octave o, as r_fm
// for a logit: 2^(y c - o) * 2^24 rounded down (yc = y c in f64).
__device__ __forceinline__ uint32_t d_pfm(double yc, int o) {
    return (uint32_t)(__builtin_amdgcn_exp2f((float)(yc - (double)o)) * 16777216.0f);
}
// PEN: the stable order on f64 values: (key64(v), row index) pairs, larger
// first; kept(v, i) <=> key > kcut or (key == kcut and i <= kidx).
__device__ __forceinline__ bool d_pkeep(unsigned long long kv, uint32_t idx, unsigned long long kcut,
                                        uint32_t kidx) {
    return (kv > kcut) | ((kv == kcut) & (idx <= kidx));
}

// Returns NIS_REJECT_NONE when the row is done, else (uniformly across the
// workgroup) why the general path must recompute it; nothing has been
// written then.
template <bool PEN>
__device__ __forceinline__ uint32_t dense_row(const RowArgs a, const int row, NucleusShared& sh) {
    const int l = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int tid = (int)threadIdx.x;
    const int V = (int)a.V;
    const gfp rowp = (gfp)(a.logits + (int64_t)row * a.ld);
    const int mis = (int)(((uintptr_t)rowp >> 2) & 3);  // elements before the row in its 16 B block
    const gf4p base = (gf4p)(rowp - mis);
    const int f_lo = mis ? 1 : 0;          // first float4 slot lying fully inside the row
    const int f_hi = (V + mis - 4) >> 2;   // last one
    const int nsl = (V + mis + 3) >> 2;    // slots touching the row
    // the row's chunks split as evenly as they go: every wave nch / kDW of
    // them, the first nch % kDW waves one more (the stream is bound by VALU
    // issue, so each SIMD's share of chunks sets its length)
    const int nch = (nsl + 63) >> 6;
    const int cb = nch / kDW, cr = nch % kDW;
    int Kw = cb + (w < cr ? 1 : 0);  // <= kDN: V <= kDMaxV
    const int wbase = 64 * (cb * w + min(w, cr));
    const int slot0 = wbase + l;
    // row index of element 0 of chunk k of this lane
#define NIS_RIDXD(k) (4 * (slot0 + 64 * (k)) - mis)
    NIS_DTDECL
    NIS_DTS(0);

    // the (at most 3 + 3) elements of partial head / tail slots, by one
    // vector load (lane i < 3: element i, lane 3 + i: element V - 6 + 3 + i)
    const float hv = rowp[(l < 3) ? l : ((l < 6) ? V - 6 + l : 0)];
    __builtin_amdgcn_sched_barrier(0);
    const uint64_t bptr = (uint64_t)(uintptr_t)base;
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    f4v xv[kDN];
    // Chunk 0 first; then the histogram ring and the counters are cleared and
    // one barrier orders that before any add.  The barrier sits before the
    // other loads: a barrier behind a wave's whole batch of loads would wait
    // until the CU has issued them all, which it does only as data arrives.
    xv[0] = nis_buffer_load_f4(rsrc, (Kw > 0) ? 16 * max(slot0, f_lo) : 0x7FFFFFF0, 0, 2);
    __builtin_amdgcn_sched_barrier(0);
    // PEN: the raw history ids (behind chunk 0), and the bitmaps cleared
    uint32_t hid[kPHist / kPB];
    // (too long a history declines the row; the flag is stored once the
    // first barrier is behind, so that no wave waits for the history's
    // length before the row's next loads go out)
    bool hlong = false;
    if constexpr (PEN) {
        hlong = pen_load_ids(a, row, tid, hid);
        pen_clear(sh.u.pb, tid);
    }
    {
        u4v* const rp = reinterpret_cast<u4v*>(&sh.ring[(kDRing / kDB) * tid]);
#pragma unroll
        for (int i = 0; i < kDRing / kDB / 2; ++i) rp[i] = u4v{0u, 0u, 0u, 0u};
    }
    if (tid < 64) sh.sub[tid] = 0ull;
    if (tid == 0) {
        sh.nmem = 0u;
        sh.over = 0u;
        sh.kmax = 0u;
        sh.krw0 = 0xFFFFFFFFu;
        sh.krw0hi = 0u;
        sh.fnan = 0u;
        if (PEN) {
            sh.kpl = 0u;
            sh.kymax = 0ull;
            sh.pover = 0u;
        }
    }
    lds_barrier();
    const int voff = 16 * slot0;  // (chunks past the first never hold slot 0)
#define NIS_DLOAD(k)                                                                          \
    do {                                                                                      \
        xv[k] = nis_buffer_load_f4(rsrc, ((k) < Kw) ? voff + 1024 * (k) : 0x7FFFFFF0, 0, 2);  \
    } while (0)
#pragma unroll
    for (int k = 1; k < kDD && k < kDN; ++k) {
        NIS_DLOAD(k);
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
        pen_set_bits(sh.u.pb, hid, V, mis);
        if (tid == 0 && hlong) atomicOr(&sh.pover, 1u);
        lds_barrier();
        pen_masks<kDN>(sh.u.pb, wbase, Kw, l, pany, pnl);
    }
    // the CU serves the waves' loads in wave order: later waves run at a
    // higher priority until their stream ends
    __builtin_amdgcn_s_setprio(0);
    if (w >= kDW / 4) __builtin_amdgcn_s_setprio(1);
    if (w >= kDW / 2) __builtin_amdgcn_s_setprio(2);
    if (w >= 3 * kDW / 4) __builtin_amdgcn_s_setprio(3);

    const bool edge_wave = (wbase < f_lo) || (wbase + 64 * Kw - 1 > f_hi);
    const float h0 = bcast_f32(hv, 0), h1 = bcast_f32(hv, 1), h2 = bcast_f32(hv, 2);
    const float t0 = bcast_f32(hv, 3), t1 = bcast_f32(hv, 4), t2 = bcast_f32(hv, 5);
    const f4v ninf4 = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#define NIS_DFIX(k)                                                                           \
    do {                                                                                      \
        if ((k) >= Kw) xv[k] = ninf4;                                                         \
        else if (edge_wave) {                                                                 \
            const int fb0 = wbase + (k) * 64;                                                 \
            if (fb0 < f_lo || fb0 + 63 > f_hi)                                                \
                xv[k] = fix_slot(xv[k], slot0 + (k) * 64, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2); \
        }                                                                                     \
    } while (0)

    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const double c64 = 1.4426950408889634 / temp;            // log2(e) / T
    // c_hi rounded toward zero, so c_lo >= 0 and x = -inf gives -inf, not NaN
    float chi = (float)c64;
    if ((double)chi > c64) chi = __uint_as_float(__float_as_uint(chi) - 1u);
    const float clo = (float)(c64 - (double)chi);
    const float chi64 = chi * 64.0f;  // exact: bucket j = floor(x * chi64) = floor(64 f32(x c_hi))
    const float p = a.top_p;
    const double pen = (double)a.penalty;
    const double chid = (double)chi;

    // ---- stream: chunk masses, max, and every element into the ring --------
    NIS_DFIX(0);
    // (PEN: of the plain elements; the stream leaves the penalised ones out)
    float m0 = wmax_f32(r_max4((PEN && (pany & 1u)) ? d_mask4(xv[0], (uint32_t)pnl & 15u) : xv[0]));
    if (m0 == -INFINITY && Kw > 1) {
        // chunk 0 holds nothing above -inf (a masked stretch): the first
        // reference comes from the wave's whole run instead, every chunk's
        // load issued now (the stream issues them again as usual), so that
        // no element of the wave lies above it or folds below a floor set
        // too high
#pragma unroll
        for (int k = kDD; k < kDN; ++k) NIS_DLOAD(k);
        float mw = -INFINITY;
#pragma unroll
        for (int k = 1; k < kDN; ++k) {
            if (k < Kw) {
                f4v t = xv[k];
                if (edge_wave) {
                    const int fb0 = wbase + k * 64;
                    if (fb0 < f_lo || fb0 + 63 > f_hi)
                        t = fix_slot(t, slot0 + k * 64, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2);
                }
                if (PEN && ((pany >> k) & 1u)) t = d_mask4(t, (uint32_t)(pnl >> (4 * k)) & 15u);
                mw = fmaxf(mw, r_max4(t));
            }
        }
        m0 = wmax_f32(mw);
    }
    const float Rw0 = (m0 > -INFINITY && fabsf(m0 * chi) < 1e30f) ? ceilf(m0 * chi) : 0.0f;
    // elements more than 64 octaves below the first reference share one bucket
    // (each lane's floor is its own bucket of the floor octave, so the adds
    // of a row's -inf entries are spread over 64 LDS addresses instead of
    // serialised on one; that octave lies 64 octaves below the wave's first
    // reference, at or below the bottom of the searched ones, and never
    // holds the cutoff at top-p < 1)
    const float tflo = (Rw0 - (float)kDSpan) * 64.0f + (float)l;
    float mx = -INFINITY;   // (PEN: of the plain elements)
    float mxu = -INFINITY;  // PEN: of the penalised values rounded up
    double ymx = -INFINITY; // PEN: of the penalised values
    // this lane's float4 masses go to sh.em4 chunk by chunk (2^R_z units):
    // the walk and the kept sums take the same values; chunks before kfin
    // were summed at an older reference and are summed again at the final
    // one below; z is the lane's total of them
    double z = 0.0;
    int kfin = 0;
    float* const em4w = &sh.em4[w][0][l];
    float czh = chi, czl = clo;
    asm volatile("" : "+v"(czh), "+v"(czl));
    float Rz = Rw0;
#pragma unroll
    for (int k = 0; k < kDN; ++k) {
        if (k + kDD < kDN) NIS_DLOAD(k + kDD);
        __builtin_amdgcn_sched_barrier(0);
        if (k >= Kw) continue;
        if (k > 0) NIS_DFIX(k);
        // PEN: the penalised elements are -inf in this copy (mass 0, count 1
        // in the floor bucket, taken back with their own adds after the stream)
        f4v x = xv[k];
        if (PEN && ((pany >> k) & 1u)) x = d_mask4(x, (uint32_t)(pnl >> (4 * k)) & 15u);
#define NIS_DHIST(jq, eq)                                                                  \
        {                                                                                  \
            const int j_ = d_flr(d_vmax((jq), tflo));                                      \
            const uint32_t fm_ = (uint32_t)__builtin_amdgcn_ldexpf((eq), Rs - (j_ >> 6));   \
            __hip_atomic_fetch_add(&sh.ring[j_ & (kDRing - 1)], (1ull << 48) | fm_,       \
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);        \
        }
        const float m4 = r_max4(x);
        mx = fmaxf(mx, m4);
        // the reference follows the running max (the total moves by the exact
        // power of two)
        if (__ballot(m4 * chi > Rz + 1.0f)) {
            const float Rn = ceilf(wmax_f32(mx) * chi);
            if (fabsf(Rn) < 1e30f) {
                Rz = Rn;
                kfin = k;
                z = 0.0;
            }
        }
        const int Rs = (int)Rz + 24;
        const float e0 = r_mass(x.x, czh, czl, Rz), e1 = r_mass(x.y, czh, czl, Rz);
        const float e2 = r_mass(x.z, czh, czl, Rz), e3 = r_mass(x.w, czh, czl, Rz);
        {
            const float s4 = (e0 + e1) + (e2 + e3);
            em4w[64 * k] = s4;
            z += (double)s4;
        }
        NIS_DHIST(x.x * chi64, e0)
        NIS_DHIST(x.y * chi64, e1)
        NIS_DHIST(x.z * chi64, e2)
        NIS_DHIST(x.w * chi64, e3)
#undef NIS_DHIST
    }
    NIS_DTS(1);
    __builtin_amdgcn_s_setprio(0);
    mx = wmax_f32(mx);
    // the masses of chunks summed before the reference last moved, again at
    // the final reference (kfin is wave-uniform and usually 0); then the
    // lane's total, NaN if any element is NaN
    if (kfin > 0) {
#pragma unroll
        for (int k = 0; k < kDN; ++k) {
            if (k < kfin) {
                f4v x = xv[k];
                if (PEN && ((pany >> k) & 1u)) x = d_mask4(x, (uint32_t)(pnl >> (4 * k)) & 15u);
                const float s4 = (r_mass(x.x, czh, czl, Rz) + r_mass(x.y, czh, czl, Rz)) +
                                 (r_mass(x.z, czh, czl, Rz) + r_mass(x.w, czh, czl, Rz));
                em4w[64 * k] = s4;
                z += (double)s4;
            }
        }
    }
    // PEN: fn(x, k) for each penalised element of this lane's own slots
    // (bit 4 k + q of pnl, in that order; few per lane): its logit x taken
    // from the registers, k its chunk.  One copy of the code, so the
    // per-element f64 work is not repeated for every register chunk.
    // (Until the cutoff search; after it each_pen reads the parked logits.)
    auto each_pen_x = [&](auto&& fn) {
        if constexpr (PEN) {
            uint64_t bits = pnl;
            while (bits) {
                const int i = __ffsll((long long)bits) - 1;
                bits &= bits - 1ull;
                const int k = i >> 2, q = i & 3;
                // (a switch: a select loop over a runtime chunk index is
                // turned into an indexed copy of xv in scratch memory, whose
                // stores in the stream wait on every load in flight)
                f4v c;
                switch (k) {
                    case 0: c = xv[0]; break;
                    case 1: c = xv[1]; break;
                    case 2: c = xv[2]; break;
                    case 3: c = xv[3]; break;
                    case 4: c = xv[4]; break;
                    case 5: c = xv[5]; break;
                    case 6: c = xv[6]; break;
                    case 7: c = xv[7]; break;
                    case 8: c = xv[8]; break;
                    case 9: c = xv[9]; break;
                    case 10: c = xv[10]; break;
                    case 11: c = xv[11]; break;
                    default: c = xv[12]; break;
                }
                static_assert(kDN == 13, "one case per register chunk");
                fn(elem(c, q), k);
            }
        }
    };
    if constexpr (PEN) {
        // The penalised elements the stream left out: their max (y rounded
        // up bounds every bucket; the exact max serves the statistics), the
        // reference raised past them if they need it (every float4 mass is
        // then summed again), then their masses into their float4s' entries
        // and Z, and their buckets, each taking back the floor bucket's count
        // its -inf added.
        each_pen_x([&](float x, int) {
            const double y = pen_value(x, pen);
            ymx = fmax(ymx, y);
            mxu = fmaxf(mxu, pen_f32_up(y));
        });
        // (each lane parks its penalised values after the search: at most
        // kDPenLane of them)
        if (__popcll(pnl) > kDPenLane) atomicOr(&sh.pover, 2u);
        const float mu = wmax_f32(mxu);
        if (mu * chi > Rz + 1.0f) {
            const float Rn = ceilf(fmaxf(mx, mu) * chi);
            if (fabsf(Rn) < 1e30f) {
                Rz = Rn;
                z = 0.0;
#pragma unroll
                for (int k = 0; k < kDN; ++k) {
                    if (k < Kw) {
                        f4v x = xv[k];
                        if ((pany >> k) & 1u) x = d_mask4(x, (uint32_t)(pnl >> (4 * k)) & 15u);
                        const float s4 = (r_mass(x.x, czh, czl, Rz) + r_mass(x.y, czh, czl, Rz)) +
                                         (r_mass(x.z, czh, czl, Rz) + r_mass(x.w, czh, czl, Rz));
                        em4w[64 * k] = s4;
                        z += (double)s4;
                    }
                }
            }
        }
        const int Rs = (int)Rz + 24;
        const int jflo = d_flr(tflo);
        each_pen_x([&](float x, int k) {
            const double y = pen_value(x, pen);
            const float ey = (float)pen_mass(y * c64, Rz);
            em4w[64 * k] += ey;
            z += (double)ey;
            const int j = d_flr(d_vmax(d_pt(y, chid) * 64.0f, tflo));
            const uint32_t fm = (uint32_t)__builtin_amdgcn_ldexpf(ey, Rs - (j >> 6));
            __hip_atomic_fetch_add(&sh.ring[j & (kDRing - 1)], (1ull << 48) | fm, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_fetch_add(&sh.ring[jflo & (kDRing - 1)], 0ull - (1ull << 48), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        });
    }
    {
        const bool nan_seen = __ballot(z != z) != 0ull;
        if (l == 0) {
            if (Kw > 0) {
                atomicMax(&sh.kmax, key32(mx == mx ? mx : -INFINITY));
                atomicMin(&sh.krw0, key32(Rw0));
                if (mx > -INFINITY || (PEN && pany != 0u)) atomicMax(&sh.krw0hi, key32(Rw0));
            }
            if (nan_seen) atomicOr(&sh.fnan, 1u);
            if (PEN && Kw > 0) atomicMax(&sh.kpl, key32(mx == mx ? mx : -INFINITY));
        }
        if (PEN) {  // (few lanes: those holding penalised elements)
            if (mxu > -INFINITY) atomicMax(&sh.kmax, key32(mxu));
            if (ymx > -INFINITY) atomicMax(&sh.kymax, key64(ymx));
        }
    }
    // the row's one draw (sampler.rs:209), made by wave 0; the advanced state
    // is stored once the row cannot be declined any more
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
    asm volatile("" : "+s"(Kw));  // (the chunk tests below recomputed, not kept live)
    // ---- B1: every wave's stream and histogram adds are done -----------------
    lds_barrier();
    NIS_DTS(2);
    const bool rv = l < kDW;
    const float M = unkey32(sh.kmax);  // (NaN when no wave holds data: declined below)
    const float R = (M > -INFINITY && fabsf(M * chi) < 1e30f) ? ceilf(M * chi) : 0.0f;
    const int Ri = (int)R;
    {
        const bool anynan = sh.fnan != 0u;
        const float rw0min = unkey32(sh.krw0);
        const float rw0hi = sh.krw0hi ? unkey32(sh.krw0hi) : -INFINITY;
        // |M c| < 4096 keeps the finest bucket index floor(64^3 x c) in range;
        // no wave may fold what lies within the searched octaves (R above
        // every first reference of a wave holding data, less than 64 octaves
        // above the lowest)
        const bool ok = (M > -INFINITY) & (M < INFINITY) & !anynan & (fabsf(M * chi) < 4096.0f) &
                        (rw0hi <= R);
        if (!ok) {
            NIS_DTFLUSH();
            return NIS_REJECT_NONFINITE;
        }
        if (PEN && sh.pover != 0u) {
            NIS_DTFLUSH();
            return NIS_REJECT_CAPACITY;  // a history past the bitmaps, or a crowded lane
        }
        if (!(R - rw0min < (float)kDSpan)) {
            // The row max lies 64 or more octaves above some wave's first
            // reference (a spike or a head far above that wave's first chunk,
            // a wave masked whole, a penalty below 1 lifting the head): that
            // wave's unfolded range reaches below the 128 octaves the ring
            // holds, and would alias into the searched ones.  The ring is
            // built again from the registers with every wave's floor at least
            // 127 octaves below R (its first reference raised to R - 63),
            // each mass at the wave's final reference; nothing above the
            // floors changes, and what lies below them is 2^-127 of the max.
            // (All waves take this branch: R and rw0min are shared.)
            lds_barrier();  // (every wave has read the values above)
            {
                u4v* const rp = reinterpret_cast<u4v*>(&sh.ring[(kDRing / kDB) * tid]);
#pragma unroll
                for (int i = 0; i < kDRing / kDB / 2; ++i) rp[i] = u4v{0u, 0u, 0u, 0u};
            }
            lds_barrier();
            const float tfl = (fmaxf(Rw0, R - (float)(kDSpan - 1)) - (float)kDSpan) * 64.0f + (float)l;
            const int Rs = (int)Rz + 24;
            auto hadd = [&](float xq) {
                const float e = r_mass(xq, czh, czl, Rz);
                const int j = d_flr(d_vmax(xq * chi64, tfl));
                const uint32_t fm = (uint32_t)__builtin_amdgcn_ldexpf(e, Rs - (j >> 6));
                __hip_atomic_fetch_add(&sh.ring[j & (kDRing - 1)], (1ull << 48) | fm, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
            };
#pragma unroll 1
            for (int k = 0; k < kDN; ++k) {
                if (k < Kw) {
                    // (PEN: the penalised elements as -inf here, moved below)
                    f4v x;
                    switch (k) {  // (a switch keeps the registers out of scratch)
                        case 0: x = xv[0]; break;
                        case 1: x = xv[1]; break;
                        case 2: x = xv[2]; break;
                        case 3: x = xv[3]; break;
                        case 4: x = xv[4]; break;
                        case 5: x = xv[5]; break;
                        case 6: x = xv[6]; break;
                        case 7: x = xv[7]; break;
                        case 8: x = xv[8]; break;
                        case 9: x = xv[9]; break;
                        case 10: x = xv[10]; break;
                        case 11: x = xv[11]; break;
                        default: x = xv[12]; break;
                    }
                    if (PEN && ((pany >> k) & 1u)) x = d_mask4(x, (uint32_t)(pnl >> (4 * k)) & 15u);
                    hadd(x.x);
                    hadd(x.y);
                    hadd(x.z);
                    hadd(x.w);
                }
            }
            if constexpr (PEN) {
                const int jfl = d_flr(tfl);
                each_pen_x([&](float x, int) {
                    const double y = pen_value(x, pen);
                    const float ey = (float)pen_mass(y * c64, Rz);
                    const int j = d_flr(d_vmax(d_pt(y, chid) * 64.0f, tfl));
                    const uint32_t fm = (uint32_t)__builtin_amdgcn_ldexpf(ey, Rs - (j >> 6));
                    __hip_atomic_fetch_add(&sh.ring[j & (kDRing - 1)], (1ull << 48) | fm, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
                    __hip_atomic_fetch_add(&sh.ring[jfl & (kDRing - 1)], 0ull - (1ull << 48),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                });
            }
            lds_barrier();
        }
    }

    // ---- cutoff search: wave w takes buckets jt0 - q, jt0 = 64 R - 256 w - 4 l
    // (descending; the 64 octaves below R, complete for every wave) ----------
    const int jt0 = 64 * Ri - 256 * w - 4 * l;
    unsigned long long bm[4];
    uint32_t bc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int j = jt0 - q;
        const unsigned long long v = sh.ring[j & (kDRing - 1)];
        bc[q] = (uint32_t)(v >> 48);
        bm[q] = d_u44(v, j >> 6, Ri);
    }
    const unsigned long long lm = (bm[0] + bm[1]) + (bm[2] + bm[3]);
    const uint32_t lcn = (bc[0] + bc[1]) + (bc[2] + bc[3]);
    const unsigned long long im = rscan_u64w(lm);
    const uint32_t ic = wscan_u32(lcn);
    if (l == 63) {
        sh.wtm[w] = im;
        sh.wtc[w] = ic;
    }
    // ---- B2: the waves' bucket totals ---------------------------------------
    lds_barrier();
    NIS_DTS(10);
    // PEN: the ring has been read; each lane parks its penalised logits in
    // its own kDPenLane words of it, in pnl's bit order, and puts -inf in
    // their register places, so every later register pass skips them
    float* const ppark = reinterpret_cast<float*>(&sh.ring[0]) + kDPenLane * tid;
    if constexpr (PEN) {
        int jp = 0;
        each_pen_x([&](float x, int) { ppark[jp++] = x; });
#pragma unroll
        for (int k = 0; k < kDN; ++k)
            if ((pany >> k) & 1u) xv[k] = d_mask4(xv[k], (uint32_t)(pnl >> (4 * k)) & 15u);
    }
    // PEN: fn(y, idx, k) for each penalised element of this lane's own slots,
    // y = pen(x) of its parked logit, idx its row index, k its chunk
    auto each_pen = [&](auto&& fn) {
        if constexpr (PEN) {
            uint64_t bits = pnl;
            int jp = 0;
            while (bits) {
                const int i = __ffsll((long long)bits) - 1;
                bits &= bits - 1ull;
                const int k = i >> 2, q = i & 3;
                fn(pen_value(ppark[jp++], pen), (uint32_t)(4 * (slot0 + 64 * k) - mis + q), k);
            }
        }
    };
    const unsigned long long wmi = rscan16_u64(rv ? sh.wtm[l] : 0ull);
    const uint32_t wci = rscan_u32(rv ? sh.wtc[l] : 0u);
    const unsigned long long Z = rbcast_u64(wmi, kDW - 1);  // 2^(R - 44) units
    const double pz = (double)p * (double)Z;
    {
        unsigned long long G = (w > 0 ? rbcast_u64(wmi, w - 1) : 0ull) + (im - lm);
        uint32_t C = (w > 0 ? bcast_u32(wci, w - 1) : 0u) + (ic - lcn);
        int jp = INT32_MAX;
        unsigned long long gp_ = 0ull;
        uint32_t np_ = 0u, cp_ = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = jt0 - q;
            if ((bc[q] != 0u) && ((double)G - d_mup(j, 0, Ri) <= pz)) {
                jp = j;
                gp_ = G;
                np_ = bc[q];
                cp_ = C;
            }
            G += bm[q];
            C += bc[q];
        }
        const uint64_t pm = __ballot(jp != INT32_MAX);
        const int Lp = pm ? 63 - __clzll((long long)pm) : 0;  // deepest: the highest lane
        if (l == Lp) sh.cand[w] = DCand{gp_, jp, np_, cp_, 0u};
    }
    // ---- B3: every wave's deepest passing bucket -----------------------------
    lds_barrier();
    const DCand cd = sh.cand[rv ? l : 0];
    const uint32_t ckey = rv ? ((uint32_t)cd.j ^ 0x80000000u) : 0xFFFFFFFFu;
    const uint32_t kbest = wmin_u32(ckey);
    if (kbest == ((uint32_t)INT32_MAX ^ 0x80000000u)) {
        NIS_DTFLUSH();
        return NIS_REJECT_WINDOW;  // (cannot happen: the top bucket always passes)
    }
    const int Lb = __ffsll((long long)__ballot(rv && ckey == kbest)) - 1;
    const int bp = (int)(kbest ^ 0x80000000u);
    const unsigned long long Gp = rbcast_u64(cd.g, Lb);
    const uint32_t nsel0 = bcast_u32(cd.n, Lb);
    const uint32_t nab0 = bcast_u32(cd.nab, Lb);
    NIS_DTS(3);

    asm volatile("" : "+s"(Kw));  // (the chunk tests below recomputed, not kept live)
    // ---- listing: float4s that may hold members of b_p, and float4s of the
    // smaller side of the cutoff --------------------------------------------
    const bool kside = nab0 + nsel0 <= (uint32_t)V - nab0;  // few kept: list the kept side
    float xl_c, xh_c;  // value bounds of b_p, widened: x in b_p => xl_c < x < xh_c
    {
        const float vl = (float)bp / chi64, vh = (float)(bp + 1) / chi64;
        xl_c = vl - fabsf(vl) * 1.0e-6f - 1.0e-30f;
        xh_c = vh + fabsf(vh) * 1.0e-6f + 1.0e-30f;
    }
    // A side with more elements than the lists have slots rarely fits (its
    // elements would have to share float4s; on c2's rows with 2-8 k of them
    // the busiest wave needs 170-400 slots of 128): such a row skips the
    // listing and works in registers.
    const uint32_t nside = kside ? nab0 + nsel0 : (uint32_t)V - nab0;
    bool brute = nside > (uint32_t)(kDL * kDW);
    uint32_t nq = 0u;  // wave-uniform list length
    if (!brute) {
        const uint32_t ent0 = lds_addr(&sh.u.l.ent[w][0]), epos0 = lds_addr(&sh.u.l.epos[w][0]);
        auto list_chunks = [&](auto&& pred) {
#pragma unroll
            for (int k = 0; k < kDN; ++k) {
                if (k < Kw) {
                    // PEN: a float4 holding a penalised element is listed on either side
                    const uint32_t pmk = PEN ? (uint32_t)(pnl >> (4 * k)) & 15u : 0u;
                    const uint64_t sk = __ballot(pred(xv[k]) | (pmk != 0u));
                    const uint32_t s = min(nq + lane_rank(sk), (uint32_t)kDL - 1u);
                    lds_put_x4_u16(sk, ent0 + 16 * s, xv[k], epos0 + 2 * s, (uint32_t)(k * 64 + l));
                    nq += (uint32_t)__popcll(sk);
                }
            }
        };
        if (kside) list_chunks([&](const f4v& x) { return r_max4(x) >= xl_c; });
        else list_chunks([&](const f4v& x) { return d_min4(x) <= xh_c; });
        if (l == 0 && nq > (uint32_t)kDL) atomicOr(&sh.over, 1u);
    }
    // ---- B4: lists complete ---------------------------------------------------
    lds_barrier();
    NIS_DTS(4);
    brute = brute || sh.over != 0u;

    asm volatile("" : "+s"(Kw));  // (the chunk tests below recomputed, not kept live)
    // ---- the cutoff bucket's members: refined while more than kDMem ----------
    // Every float4 holding a member of b_p is on the listed side (or, when a
    // list overflowed, in this lane's registers); fn(x4, i0, valid) visits
    // them, i0 the row index of element 0 (PEN: the penalised elements are
    // -inf there; each_pen visits them).
    const int ne = (int)min(nq, (uint32_t)kDL);
    auto each_float4 = [&](auto&& fn) {
        if (!brute) {
#pragma unroll
            for (int r = 0; r < kDL / 64; ++r) {
                if (64 * r < ne) {
                    const int je = 64 * r + l;
                    fn(sh.u.l.ent[w][je], (uint32_t)(4 * (wbase + (int)sh.u.l.epos[w][je]) - mis),
                       je < ne);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < kDN; ++k)
                if (k < Kw) fn(xv[k], (uint32_t)NIS_RIDXD(k), true);
        }
    };
    int lv = 0, B = bp;
    unsigned long long Gc = Gp;
    uint32_t ns = nsel0, nabv = nab0;
    float chiL = chi64;
    float scL = 64.0f;  // 64^(lv + 1): the level's buckets of T(v)
    bool all_out = false;  // the whole bucket is removed (no sub-bucket passes)
    while (ns > (uint32_t)kDMem) {
        if (lv == kDLevels - 1) {
            NIS_DTFLUSH();
            return NIS_REJECT_CAPACITY;  // exact ties beyond kDMem members
        }
        const int o = B >> (6 * (lv + 1));  // the bucket's octave
        const float chiS = chiL * 64.0f, scS = scL * 64.0f;
        each_float4([&](const f4v& x4, uint32_t i0, bool valid) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float x = elem(x4, q);
                const bool mem = valid & (d_flr(x * chiL) == B);
                if (__ballot(mem)) {
                    const uint32_t fm = r_fm(x, chi, clo, o);
                    const uint32_t sb = (uint32_t)d_flr(x * chiS) & 63u;
                    if (mem)
                        __hip_atomic_fetch_add(&sh.sub[sb], (1ull << 48) | (unsigned long long)fm,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        });
        each_pen([&](double y, uint32_t, int) {
            const float t = d_pt(y, chid);
            if (d_flr(t * scL) == B)
                __hip_atomic_fetch_add(&sh.sub[(uint32_t)d_flr(t * scS) & 63u],
                                       (1ull << 48) | (unsigned long long)d_pfm(y * c64, o), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
        });
        lds_barrier();
        if (w == 0) {
            // lane l takes sub-bucket 63 - l (descending)
            const unsigned long long v = sh.sub[63 - l];
            const uint32_t n = (uint32_t)(v >> 48);
            const unsigned long long m = d_u44(v, o, Ri);
            const unsigned long long Gs = Gc + (rscan_u64w(m) - m);
            const uint32_t Cs = nabv + (wscan_u32(n) - n);
            const int Fs = 64 * B + 63 - l;
            const uint64_t ps = __ballot((n != 0u) && ((double)Gs - d_mup(Fs, lv + 1, Ri) <= pz));
            DCut c;
            c.kcut = ~0ull;
            c.kidx = 0u;
            c.rej = 0u;
            c.nkept = 0u;
            if (ps) {
                const int Ls = 63 - __clzll((long long)ps);
                c.bj = 64 * B + 63 - Ls;
                c.lv = lv + 1;
                c.g = rbcast_u64(Gs, Ls);
                c.nsel = bcast_u32(n, Ls);
                c.nab = bcast_u32(Cs, Ls);
            } else {
                c.bj = B;
                c.lv = lv;
                c.g = Gc;
                c.nsel = 0u;  // every member of B is removed
                c.nab = nabv;
                c.rej = 1u;
            }
            sh.sub[l] = 0ull;  // (read above by lane 63 - l; clears for the next level)
            if (l == 0) sh.cut = c;
        }
        lds_barrier();
        const DCut c = sh.cut;
        B = c.bj;
        lv = c.lv;
        Gc = c.g;
        ns = c.nsel;
        nabv = c.nab;
        if (c.rej) {
            all_out = true;
            break;
        }
        chiL = chiS;
        scL = scS;
    }
    NIS_DTS(11);
    // members of the final bucket B (at most kDMem) into sh.mem
    if (!all_out && ns > 0u) {
        const int o = B >> (6 * (lv + 1));
        each_float4([&](const f4v& x4, uint32_t i0, bool valid) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float x = elem(x4, q);
                const bool mem = valid & (d_flr(x * chiL) == B);
                const uint64_t mb = __ballot(mem);
                if (mb) {
                    uint32_t b0 = 0u;
                    if (l == 0) b0 = atomicAdd(&sh.nmem, (uint32_t)__popcll(mb));
                    const uint32_t sm = bcast_u32(b0, 0) + lane_rank(mb);
                    if (mem) sh.mem[min(sm, (uint32_t)kDMem - 1u)] = RCand{x, i0 + (uint32_t)q, o, r_fm(x, chi, clo, o)};
                }
            }
        });
        each_pen([&](double y, uint32_t idx, int) {
            if (d_flr(d_pt(y, chid) * scL) == B) {
                const uint32_t sm = min(atomicAdd(&sh.nmem, 1u), (uint32_t)kDMem - 1u);
                sh.mem[sm] = RCand{0.0f, idx | 0x80000000u, o, d_pfm(y * c64, o)};
                sh.my[sm] = y;
            }
        });
    }
    lds_barrier();
    NIS_DTS(5);
    if (!all_out && sh.nmem != ns) {
        NIS_DTFLUSH();
        return NIS_REJECT_BUCKET;
    }
    // ---- rank the members (wave 0): stable descending order of sampler.rs:140
    if (w == 0) {
        DCut c;
        c.bj = B;
        c.lv = lv;
        c.g = Gc;
        c.nab = nabv;
        c.nsel = ns;
        c.rej = 0u;
        c.kcut = ~0ull;
        c.kidx = 0u;
        c.nkept = 0u;
        if (!all_out) {
            const int n = (int)ns;
            const bool valid = l < n;
            const RCand mr = sh.mem[min(l, kDMem - 1)];
            // PEN: (key64 of the value, row index) pairs
            const uint32_t im = PEN ? (mr.idx & 0x7FFFFFFFu) : mr.idx;
            unsigned long long Km;
            if constexpr (PEN)
                Km = valid ? key64((mr.idx >> 31) ? sh.my[min(l, kDMem - 1)] : (double)mr.x) : 0ull;
            else
                Km = valid ? r_key(mr.x, mr.idx) : 0ull;
            const unsigned long long em = valid ? d_u44(mr.fm, mr.b, Ri) : 0ull;
            // every lane compares its key with all of them, read back from LDS
            // (same address in every lane; eight reads in flight per step)
            sh.mkey[l] = Km;
            sh.mmass[l] = em;
            if (PEN) sh.midx[l] = im;
            lds_wave_fence();
            unsigned long long pre = 0ull;  // mass of the members ahead of this one
            uint32_t rk = 0u;
            for (int j0 = 0; j0 < n; j0 += 8) {
                unsigned long long kj[8], ej[8];
                uint32_t ij[8];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    kj[jj] = sh.mkey[min(j0 + jj, kDMem - 1)];
                    ej[jj] = sh.mmass[min(j0 + jj, kDMem - 1)];
                    ij[jj] = PEN ? sh.midx[min(j0 + jj, kDMem - 1)] : 0u;
                }
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const bool gt = PEN ? ((kj[jj] > Km) | ((kj[jj] == Km) & (ij[jj] < im))) : (kj[jj] > Km);
                    const bool ahead = (j0 + jj < n) & gt;
                    pre += ahead ? ej[jj] : 0ull;
                    rk += ahead ? 1u : 0u;
                }
            }
            // sampler.rs:150 in rank order: D = G + pre - e; the kept ones are
            // the longest prefix of ranks with D <= p Z
            const bool pass = valid & ((double)(Gc + pre) - (double)em <= pz);
            uint32_t nkept = (uint32_t)n;
            if (__ballot(valid & !pass)) nkept = wmin_u32((valid && !pass) ? rk : 0xFFFFFFFFu);
            const uint64_t lastm = __ballot(valid & (rk + 1u == nkept));
            c.kcut = lastm ? rbcast_u64(Km, __ffsll((long long)lastm) - 1) : ~0ull;
            c.kidx = lastm ? bcast_u32(im, __ffsll((long long)lastm) - 1) : 0u;
            c.nkept = nkept;
        }
        if (l == 0) sh.cut = c;
    }
    // ---- B5: the cutoff is known ----------------------------------------------
    lds_barrier();
    NIS_DTS(6);
    const DCut cut = sh.cut;
    const int Bf = cut.bj;
    const unsigned long long kcut = cut.kcut;
    const uint32_t kidx = cut.kidx;
    {
        // chi at the final level's resolution (exact powers of two)
        float cl = chi64, sl = 64.0f;
        for (int i = 0; i < cut.lv; ++i) {
            cl *= 64.0f;
            sl *= 64.0f;
        }
        chiL = cl;
        scL = sl;
    }

    asm volatile("" : "+s"(Kw));  // (the chunk tests below recomputed, not kept live)
    // ---- kept masses: this wave's listed float4s, or all of its float4s -----
    // kept mass of float4 x4 (elements 0..3 at row index i0) and its stream
    // mass, from the same per-element masses the stream summed
    // (the stable-order key is compared only in a chunk holding an element
    // of the final bucket: at most kDMem of them in the row)
    // (PEN: the penalised elements, -inf here, count 0: each_pen adds their
    // kept masses after)
    auto kept4 = [&](const f4v& x4, uint32_t i0, float& all) {
        float e[4], k4[4];
        int F[4];
        bool inb = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float x = elem(x4, q);
            e[q] = r_mass(x, czh, czl, Rz);
            F[q] = d_flr(x * chiL);
            k4[q] = (F[q] > Bf) ? e[q] : 0.0f;
            inb |= F[q] == Bf;
        }
        if (__ballot(inb)) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (F[q] != Bf) continue;
                bool kq;
                if constexpr (PEN) {
                    kq = d_pkeep(key64((double)elem(x4, q)), i0 + (uint32_t)q, kcut, kidx);
                } else {
                    kq = r_key(elem(x4, q), i0 + (uint32_t)q) >= kcut;
                }
                if (kq) k4[q] = e[q];
            }
        }
        all = (e[0] + e[1]) + (e[2] + e[3]);
        return (k4[0] + k4[1]) + (k4[2] + k4[3]);
    };
    double tws = 0.0;  // this lane's part of the wave's kept mass (2^R_z units)
    float kvb[kDN];    // brute: this lane's float4 kept masses
#pragma unroll
    for (int k = 0; k < kDN; ++k) kvb[k] = 0.0f;
    if (!brute) {
        // The parked float4 masses ([chunk][lane] of this wave) become kept
        // masses: a listed float4 takes its own; off the list every float4 is
        // kept whole (listed removed side) or removed (listed kept side).
        float* const esw = &sh.em4[w][0][0];
        if (kside) {
#pragma unroll
            for (int k = 0; k < kDN; ++k) esw[64 * k + l] = 0.0f;
            lds_wave_fence();
        }
#pragma unroll
        for (int r = 0; r < kDL / 64; ++r) {
            if (64 * r < ne) {
                const int je = 64 * r + l;
                const bool valid = je < ne;
                float orig;
                const int ep = (int)sh.u.l.epos[w][min(je, kDL - 1)];
                const float ks = kept4(sh.u.l.ent[w][min(je, kDL - 1)], (uint32_t)(4 * (wbase + ep) - mis), orig);
                if (valid) esw[ep] = ks;
                tws += valid ? (kside ? (double)ks : (double)ks - (double)orig) : 0.0;
            }
        }
        if (!kside) tws += z;  // every float4 off the list is kept whole
    } else {
        // (kept in registers: the chosen wave's walk takes them as they are)
#pragma unroll
        for (int k = 0; k < kDN; ++k) {
            if (k < Kw) {
                float orig;
                kvb[k] = kept4(xv[k], (uint32_t)NIS_RIDXD(k), orig);
                tws += (double)kvb[k];
            }
        }
    }
    if constexpr (PEN) {
        // the penalised elements' kept masses join their float4s' entries (a
        // brute row's register masses are parked there first) and the total
        float* const esw = &sh.em4[w][0][0];
        if (brute) {
#pragma unroll
            for (int k = 0; k < kDN; ++k) esw[64 * k + l] = kvb[k];
        }
        lds_wave_fence();
        const bool off_kept = !brute && !kside;  // their stream masses are already in tws
        each_pen([&](double y, uint32_t idx, int k) {
            const float ey = (float)pen_mass(y * c64, Rz);
            const int F = d_flr(d_pt(y, chid) * scL);
            const float ky = ((F > Bf) | ((F == Bf) & d_pkeep(key64(y), idx, kcut, kidx))) ? ey : 0.0f;
            esw[64 * k + l] += ky;
            tws += (double)ky - (off_kept ? (double)ey : 0.0);
        });
    }
    {
        const double Tw = wsum_f64(tws);
        if (l == 0) sh.tw[w] = ldexp(Tw, (int)(Rz - R));  // 2^R units (exact)
    }
    if (w == 0 && l < 4) a.rng[4 * (int64_t)row + l] = rst;
    asm volatile("" : "+s"(Kw));  // (the chunk tests below recomputed, not kept live)
    // ---- B6: per-wave kept masses -----------------------------------------------
    lds_barrier();
    NIS_DTS(7);
    const double T = rv ? sh.tw[l] : 0.0;
    const double Tincl = rscan16_f64(T);
    const double Zk = bcast_f64(Tincl, 15);
    const double u = sh.u0;
    const double r = u * Zk;
    // the chosen wave: the first whose inclusive total reaches r (the last
    // with mass if rounding leaves r above every prefix)
    const uint64_t hw = __ballot(rv & (T > 0.0) & (Tincl >= r));
    const uint64_t nzw = __ballot(rv & (T > 0.0));
    const int ws = hw ? (__ffsll((long long)hw) - 1) : (63 - __clzll((long long)(nzw | 1ull)));
    if (w != ws) {
        NIS_DTFLUSH();
        return NIS_REJECT_NONE;
    }
    // r inside this wave, in 2^R_z units
    const double rw_ = ldexp(r - bcast_f64(Tincl - T, ws), (int)(R - Rz));
    // this lane's per-float4 kept masses (2^R_z units), transposed into chunk
    // totals
    // this lane's float4 kept masses: in registers (brute), else the parked
    // array the kept sums left behind (one read each, all issued together)
    float kv[kDN];
    {
        const float* const esw = &sh.em4[w][0][l];
#pragma unroll
        for (int k = 0; k < kDN; ++k) kv[k] = esw[64 * k];
#pragma unroll
        for (int k = 0; k < kDN; ++k) kv[k] = (brute && !PEN) ? kvb[k] : ((k < Kw) ? kv[k] : 0.0f);
    }
#pragma unroll
    for (int k = 0; k < kDN; ++k) sh.walk[k][l] = kv[k];
    NIS_DTS(14);
    lds_wave_fence();
    // lane j < 4 kDN: quarter j & 3 of chunk j >> 2
    double qs = 0.0;
    if (l < 4 * kDN) {
        const int kk = l >> 2, qq = l & 3;
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const f4v v = *reinterpret_cast<const f4v*>(&sh.walk[kk][16 * qq + i]);
            qs += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
        }
    }
    {
        const uint64_t b_ = (uint64_t)__double_as_longlong(qs);
        const uint64_t lo_ = dpp0<0x111, 0xF>((uint32_t)b_), hi_ = dpp0<0x111, 0xF>((uint32_t)(b_ >> 32));
        qs += __longlong_as_double((long long)((hi_ << 32) | lo_));
    }
    {
        const uint64_t b_ = (uint64_t)__double_as_longlong(qs);
        const uint64_t lo_ = dpp0<0x112, 0xF>((uint32_t)b_), hi_ = dpp0<0x112, 0xF>((uint32_t)(b_ >> 32));
        qs += __longlong_as_double((long long)((hi_ << 32) | lo_));  // lane 4i+3: chunk i
    }
    const double ck = __shfl(qs, 4 * min(l, kDN - 1) + 3);
    const double cks = (l < kDN && l < Kw) ? ck : 0.0;
    const double cincl = rscan16_f64(cks);  // kDN <= 16: one DPP row
    const uint64_t hk = __ballot((l < 16) & (cks > 0.0) & (cincl >= rw_));
    const uint64_t nzk = __ballot((l < 16) & (cks > 0.0));
    const int kc = hk ? (__ffsll((long long)hk) - 1) : (63 - __clzll((long long)(nzk | 1ull)));
    NIS_DTS(15);
    const double rk_ = rw_ - bcast_f64(cincl - cks, kc);
    // the lanes of chunk kc in index order
    f4v xc = xv[0];
    float sc = kv[0];
#pragma unroll
    for (int k = 1; k < kDN; ++k)
        if (k == kc) {
            xc = xv[k];
            sc = kv[k];
        }
    const double sl = (double)sc;
    const double lincl = wscan_f64(sl);
    const uint64_t hl = __ballot((sl > 0.0) & (lincl >= rk_));
    const uint64_t nzl = __ballot(sl > 0.0);
    const int lc = hl ? (__ffsll((long long)hl) - 1) : (63 - __clzll((long long)(nzl | 1ull)));
    NIS_DTS(8);
    if (l == lc) {
        double run = rk_ - (lincl - sl);
        const uint32_t ib = (uint32_t)NIS_RIDXD(kc);
        const uint32_t pmc = PEN ? (uint32_t)(pnl >> (4 * kc)) & 15u : 0u;
        float ev[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float xq = elem(xc, q);
            // the same masses the float4's kept total was summed from
            // (a float4 kept whole passes every test: its elements lie above b_p)
            if constexpr (PEN) {
                // (a penalised element's logit is parked: the j-th set bit of pnl)
                const bool pq = (pmc >> q) & 1u;
                const double v =
                    pq ? pen_value(ppark[__popcll(pnl & ((1ull << (4 * kc + q)) - 1ull))], pen) : (double)xq;
                const float eq = pq ? (float)pen_mass(v * c64, Rz) : r_mass(xq, czh, czl, Rz);
                const int F = pq ? d_flr(d_pt(v, chid) * scL) : d_flr(xq * chiL);
                ev[q] = ((F > Bf) | ((F == Bf) & d_pkeep(key64(v), ib + (uint32_t)q, kcut, kidx))) ? eq : 0.0f;
            } else {
                const float eq = r_mass(xq, czh, czl, Rz);
                ev[q] = d_kept(xq, ib + (uint32_t)q, chiL, Bf, kcut) ? eq : 0.0f;
            }
        }
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
        uint32_t tok = ib + (uint32_t)q;
        if (u == 0.0) tok = 0u;  // r == 0 stops the reference's walk at index 0
        emit_token(a, row, tok);
        if (a.stats) {
            // PEN: the exact max over the plain and the penalised values, and
            // the drawn token's value after the penalty
            const double Mx = PEN ? fmax((double)unkey32(sh.kpl), unkey64(sh.kymax)) : (double)M;
            const double vq = (PEN && ((pmc >> q) & 1u))
                                  ? pen_value(ppark[__popcll(pnl & ((1ull << (4 * kc + q)) - 1ull))], pen)
                                  : (double)xq;
            // 2^(R - M c): units of 2^R -> units of the max element's mass
            const double rho = exp2((double)R - Mx * c64);
            const double em = exp2(vq * c64 - Mx * c64);
            const double zM = Zk * rho;
            write_row_stats(a, row, tok, NIS_PATH_DRAW, Mx / temp, zM,
                            (double)Z / 17592186044416.0 * rho, u, (u == 0.0) ? 0.0 : em / zM,
                            (uint64_t)(cut.nab + cut.nkept), 1);
        }
    }
    NIS_DTS(9);
    NIS_DTFLUSH();
    return NIS_REJECT_NONE;
#undef NIS_DLOAD
#undef NIS_DFIX
#undef NIS_RIDXD
}

union DenseKernelShared {
    GeneralShared g;
    NucleusShared d;
};

// One 1024-lane workgroup per row: the dense path, or the general path (on
// the first 512 lanes) for a row it declines or cannot take.
template <bool PEN>
__device__ __forceinline__ void dense_kernel(const RowArgs a, DenseKernelShared& sh) {
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;  // a finished sequence (decode step)
    asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.temperature), "s"(a.top_p),
                 "s"(a.penalty), "s"(a.gen_ids), "s"(a.gen_off));
    uint32_t reject = NIS_REJECT_SHAPE;
    if (dense_eligible<PEN>(a, row)) {
        reject = dense_row<PEN>(a, row, sh.d);
        if (reject == NIS_REJECT_NONE) return;
    }
    if (threadIdx.x >= kBlock) return;
    __syncthreads();
    general_row<1>(a, row, sh.g, reject);
}

__global__ __launch_bounds__(kDB) void sample_rows_dense_kernel(RowArgs a) {
    __shared__ DenseKernelShared sh;
    dense_kernel<false>(a, sh);
}

// The same with a repetition-penalty history applied in registers.
__global__ __launch_bounds__(kDB) void sample_rows_dense_pen_kernel(RowArgs a) {
    __shared__ DenseKernelShared sh;
    dense_kernel<true>(a, sh);
}

}  // namespace nis
