// long_path.h — rows too long for the registers (53245 < V <= 2^20): one row
// per 512-lane workgroup (8 wave64s, two workgroups per CU), streamed once from
// HBM; the passes after the stream read the row again (it was just read, so
// from L2 / the memory-side cache) instead of holding it (src/sampler.rs:163-
// 216).
//
// Layout as in the register-resident kernels: wave w owns the contiguous
// 64-slot chunks [cpw w, cpw (w + 1)) of the row's float4 slots, lane l of
// chunk k holds slot 64 (cpw w + k) + l, so index order inside a wave is
// chunk, lane, element.  Every lane keeps kLD loads in flight.
//
// Greedy (sampler.rs:172-181): the first index of the maximum, one pass.
// Top-p off: the masses 2^(x c - R_z) summed per wave in the stream; the
// wave holding the draw reads its chunks again and walks them.
// Top-p (sampler.rs:118-160), any nucleus size: the method of the dense
// kernel (dense_path.h).  Every element joins one exact histogram in the
// stream (1/64-octave buckets of f32(x c_hi) on an absolute grid, count and
// octave-relative fixed-point mass; a ring of 4096 buckets, elements more
// than 32 octaves below a wave's first reference folded into one bucket);
// one block-wide scan finds the deepest bucket b_p with G(b) - m_up(b) <=
// p Z within 32 octaves of R; its members are refined to at most 64 and
// ranked exactly.  The smaller side of the cutoff is then listed by a second
// read of the row and recomputed one float4 per lane (every float4 again
// when a list overflows); the walk goes waves -> the chosen wave's listed
// float4s (few kept) or its chunks read a third time (few removed) ->
// lanes -> elements.
//
// A row this path cannot prove returns a reject code before anything is
// written, and the caller runs the general path on it.
#pragma once
#include "dense_path.h"

namespace nis {

constexpr int kLB = 512;              // lanes per workgroup (two workgroups share a CU)
constexpr int kLW = kLB / 64;         // waves per workgroup
constexpr int kLD = 4;                // loads in flight per lane
constexpr int kLRing = 4096;          // histogram ring: 64 octaves of 64 buckets
constexpr int kLSpan = 32;            // octaves searched below R (and folded below R_w0)
constexpr int kLQ = 64 * kLSpan / kLB;  // searched buckets per lane
constexpr uint32_t kLPending = 0xFFF00000u;  // token of a declined row (| reject code)
constexpr int kLMem = 2048;           // members of the cutoff bucket listed by the second read

enum { kLongTopP = 0, kLongAll = 1, kLongGreedy = 2 };
constexpr int kLPenMaxV = kLRing * 64 - 64;  // greedy with a penalty history: the bitmap's reach

// A member of the cutoff bucket, listed by the second read.
struct LMem {
    float x;
    uint32_t idx;
};

struct LongShared {
    unsigned long long ring[kLRing];  // [j & (kLRing - 1)]: count << 48 | sum of fm
    LMem lmem[kLMem];                 // the cutoff bucket's members (second read)
    RCand mem[kDMem];                 // members of the final bucket
    unsigned long long sub[64];       // refinement histogram of the cutoff bucket
    DRec rec[kLW];
    unsigned long long wtm[kLW];      // search: each wave's bucket mass
    unsigned long long wlo[kLW];      //   and that of the 32 octaves below the search
    uint32_t wtc[kLW];                //   and count
    DCand cand[kLW];
    double tw[kLW];                   // per-wave kept mass (2^R units)
    double tmem[kLW];                 // per-wave kept mass of listed members (2^R_z units)
    uint32_t nfin[kLW];               // top-p off: each wave's elements above -inf (stats)
    double gx[kLW];                   // greedy: each wave's max (penalised values in f64)
    int32_t gi[kLW];                  //   and the first index holding it
    DCut cut;
    double u0;                        // the draw
    uint32_t nmem;                    // members listed by the second read
    uint32_t cnt;                     // members of the final bucket
};

template <int MODE>
__device__ __forceinline__ bool long_eligible(const RowArgs a, int row) {
    if (a.V < 256 || a.V > NIS_MAX_V) return false;
    if (MODE == kLongGreedy) {
        if (!(a.temperature <= 0.0f)) return false;
    } else {
        if (!(a.temperature > 0.0f) || (a.top_k > 0 && a.top_k < (uint64_t)a.V)) return false;
        if (MODE == kLongAll ? !(a.top_p >= 1.0f) : !(a.top_p > 0.0f && a.top_p < 1.0f)) return false;
    }
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1) && g1 > g0) {
        // greedy and top-p off take the history as a bitmap over the ring's words
        if (MODE == kLongTopP || a.V > kLPenMaxV) return false;
    }
    return true;
}

// Returns NIS_REJECT_NONE when the row is done, else (uniformly across the
// workgroup) why the general path must recompute it; nothing has been
// written then.  `prior`: why the single-read path (long_sparse_path.h)
// declined the row, when this runs after it (reported in the row's stats).
//
// Top-p: a row whose max lies kLSpan or more octaves above a wave's first
// reference (a forced token, a masked wave under high logits) would alias in
// the ring.  With `rnext` given, such a row returns kLSpanRetry and *rnext =
// R - (kLSpan - 1); run again with rfloor = *rnext (every first reference
// raised to at least that), it fits.
constexpr uint32_t kLSpanRetry = 0x200u;  // (internal: never reported)
constexpr uint32_t kLSpanFlag = 0x40000u; // pending token: retry with rfloor in the low 14 bits (+8192)
template <int MODE>
__device__ __forceinline__ uint32_t long_row(const RowArgs a, const int row, LongShared& sh,
                                             uint32_t prior = NIS_REJECT_NONE, const float rfloor = -INFINITY,
                                             float* const rnext = nullptr) {
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
    const int cpw = (((nsl + 63) >> 6) + kLW - 1) / kLW;  // chunks per wave
    const int wbase = 64 * cpw * w;
    const int Kw = min(max((nsl - wbase + 63) >> 6, 0), cpw);
    const int slot0 = wbase + l;
    // row index of element 0 of chunk k of this lane
#define NIS_LIDX(k) (4 * (slot0 + 64 * (k)) - mis)
    NIS_DTDECL
    NIS_DTS(0);

    const float hv = rowp[(l < 3) ? l : ((l < 6) ? V - 6 + l : 0)];
    __builtin_amdgcn_sched_barrier(0);
    const uint64_t bptr = (uint64_t)(uintptr_t)base;
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    // chunk k of this lane as loaded (slot 0 of a misaligned row is read from
    // slot f_lo instead; chunks past the wave's read zeros): fixed below
    auto ld = [&](int k) -> f4v {
        const int s = slot0 + 64 * k;
        return nis_buffer_load_f4(rsrc, (k < Kw) ? 16 * max(s, f_lo) : 0x7FFFFFF0, 0, 2);
    };
    const float h0 = bcast_f32(hv, 0), h1 = bcast_f32(hv, 1), h2 = bcast_f32(hv, 2);
    const float t0 = bcast_f32(hv, 3), t1 = bcast_f32(hv, 4), t2 = bcast_f32(hv, 5);
    const f4v ninf4 = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    // the row's values of chunk k (outside the row: -inf)
    auto fixc = [&](f4v v, int k) -> f4v {
        if (k >= Kw) return ninf4;
        const int fb0 = wbase + 64 * k;
        if (fb0 < f_lo || fb0 + 63 > f_hi)
            return fix_slot(v, slot0 + 64 * k, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2);
        return v;
    };

    f4v buf[kLD];
    buf[0] = ld(0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MODE == kLongTopP) {
        u4v* const rp = reinterpret_cast<u4v*>(&sh.ring[(kLRing / kLB) * tid]);
#pragma unroll
        for (int i = 0; i < kLRing / kLB / 2; ++i) rp[i] = u4v{0u, 0u, 0u, 0u};
        if (tid < 64) sh.sub[tid] = 0ull;
        if (tid == 0) sh.nmem = 0u;
        lds_barrier();
    }
#pragma unroll
    for (int i = 1; i < kLD; ++i) {
        buf[i] = ld(i);
        __builtin_amdgcn_sched_barrier(0);
    }
    typedef const __attribute__((address_space(1))) uint64_t* gu64p;
    uint64_t rsv = 0;
    if (MODE != kLongGreedy && w == 0) rsv = ((gu64p)(a.rng + 4 * (int64_t)row))[l & 3];

    // ---- greedy and top-p off: a repetition-penalty history (sampler.rs:
    // 83-101) becomes a bitmap of the row's indices over the ring's words
    // (V <= kLPenMaxV); pnib(i0) is the 4-bit mask of indices i0 .. i0 + 3
    // (i0 >= -3; indices outside the row are -inf in the stream and set no
    // bit)
    int64_t pg0 = 0, pg1 = 0;
    const bool pen = MODE != kLongTopP && a.penalty != 1.0f && gen_range(a, row, pg0, pg1) &&
                     pg1 > pg0;  // (uniform)
    uint32_t* const pbm = reinterpret_cast<uint32_t*>(&sh.ring[0]);
    if (pen) {
        const int nwd = ((int)a.V + 31) / 32 + 1;  // (+1: the window's second word)
        for (int i = tid; i < nwd; i += kLB) pbm[i] = 0u;
        lds_barrier();
        for (int64_t i = pg0 + tid; i < pg1; i += kLB) {
            const uint32_t id = a.gen_ids[i];
            if (id < (uint32_t)a.V) atomicOr(&pbm[id >> 5], 1u << (id & 31));
        }
        lds_barrier();
    }
    const double penf = (double)a.penalty;
    auto pnib = [&](int i0) -> uint32_t {
        const int ib = max(i0, 0);
        const uint32_t wd = (uint32_t)ib >> 5;
        const unsigned long long win = (unsigned long long)pbm[wd] | ((unsigned long long)pbm[wd + 1] << 32);
        uint32_t nb = (uint32_t)(win >> (ib & 31)) & 15u;
        if (i0 < 0) nb = (nb << (-i0)) & 15u;
        return nb;
    };

    // =====================================================================
    if constexpr (MODE == kLongGreedy) {
        // ---- greedy: first index of the maximum (sampler.rs:172-181) ----
        // A float4 holding a penalised element takes its f64 values aside
        // (the lane's own max and first index) and -inf in their places.
        float bx = -INFINITY;
        int bi = 0x7FFFFFFF;
        double by = -INFINITY;  // the lane's penalised max (above -inf) and its first index
        int byi = 0x7FFFFFFF;
        float fs = 0.0f;  // NaN probe (of the logits, penalised ones included)
        // (two copies of the stream: the plain one keeps the loop of a row
        // without a history as lean as it was)
        auto stream = [&](auto PEN_) {
        constexpr bool PENS = decltype(PEN_)::value;
        for (int k0 = 0; k0 < Kw; k0 += kLD) {
#pragma unroll
            for (int i = 0; i < kLD; ++i) {
                const int k = k0 + i;
                f4v x = fixc(buf[i], k);
                buf[i] = ld(k + kLD);
                if (k < Kw) {
                    fs += (x.x + x.y) + (x.z + x.w);
                    if constexpr (PENS) {
                        const int i0 = NIS_LIDX(k);
                        const uint32_t nb = pnib(i0);
                        if (nb) {
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                if ((nb >> q) & 1u) {
                                    const double y = pen_value(elem(x, q), penf);
                                    if (y > -INFINITY && (y > by || (y == by && i0 + q < byi))) {
                                        by = y;
                                        byi = i0 + q;
                                    }
                                }
                            }
                            x = f4v{(nb & 1u) ? -INFINITY : x.x, (nb & 2u) ? -INFINITY : x.y,
                                    (nb & 4u) ? -INFINITY : x.z, (nb & 8u) ? -INFINITY : x.w};
                        }
                    }
                    const float m4 = r_max4(x);
                    const int q = (x.x == m4) ? 0 : ((x.y == m4) ? 1 : ((x.z == m4) ? 2 : 3));
                    const bool up = m4 > bx;
                    bi = up ? NIS_LIDX(k) + q : bi;
                    bx = up ? m4 : bx;
                }
            }
        }
        };
        if (pen) stream(std::true_type{});
        else stream(std::false_type{});
        // the lane's best in f64 (plain and penalised), the first index at it
        const double vb = fmax((double)bx, by);
        const uint32_t ib2 = min((uint32_t)(((double)bx == vb) ? bi : 0x7FFFFFFF),
                                 (uint32_t)((by == vb) ? byi : 0x7FFFFFFF));
        double wm = vb;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) wm = fmax(wm, __shfl_xor(wm, o));
        const int wi = (int)wmin_u32((vb == wm) ? ib2 : 0x7FFFFFFFu);
        const uint32_t bad = (uint32_t)(__ballot(fs != fs) != 0ull);
        if (l == 0) {
            sh.gx[w] = wm;
            sh.gi[w] = bad ? -1 : wi;
        }
        lds_barrier();
        const bool rv = l < kLW;
        const double gx = rv ? sh.gx[l] : -INFINITY;
        const int gi = rv ? sh.gi[l] : 0x7FFFFFFF;
        if (__ballot(rv & (gi < 0))) return NIS_REJECT_NONFINITE;
        double M = gx;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) M = fmax(M, __shfl_xor(M, o));
        int tok = (int)wmin_u32((uint32_t)((rv && gx == M) ? gi : 0x7FFFFFFF));
        if (tok == 0x7FFFFFFF) tok = 0;  // every element -inf: nothing exceeds work[0]
        if (w == 0 && l == 0)
            write_row_result(a, row, (uint32_t)tok, NIS_PATH_GREEDY, M, 0.0, 0.0, -1.0, 0.0, 0, 1);
        return NIS_REJECT_NONE;
    }

    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const double c64 = 1.4426950408889634 / temp;            // log2(e) / T
    float chi = (float)c64;
    if ((double)chi > c64) chi = __uint_as_float(__float_as_uint(chi) - 1u);
    const float clo = (float)(c64 - (double)chi);
    const float chi64 = chi * 64.0f;
    float czh = chi, czl = clo;
    asm volatile("" : "+v"(czh), "+v"(czl));

    // ---- stream -----------------------------------------------------------
    const float m0 = wmax_f32(r_max4(fixc(buf[0], 0)));
    const float Rw0 = fmaxf((m0 > -INFINITY && fabsf(m0 * chi) < 1e30f) ? ceilf(m0 * chi) : 0.0f, rfloor);
    const float tflo = (Rw0 - (float)kLSpan) * 64.0f;  // deeper elements share one bucket
    float Rz = Rw0;
    float mx = -INFINITY;  // (top-p off with a penalty: penalised values rounded up)
    double mex = -INFINITY; // top-p off with a penalty: the exact max (statistics)
    double z = 0.0;     // the lane's mass total (2^R_z units)
    uint32_t nfin = 0;  // top-p off with stats: elements above -inf (the kept count)
    // Top-p off with a penalty: the f64 values y of a float4's penalised
    // elements give the max operand pen_f32_up(y) and the masses
    // 2^(y c - R_z) in place of their logits'.  (Two copies of the stream:
    // a row without a history keeps the plain one.)
    auto sstream = [&](auto PEN_) {
    constexpr bool PENS = decltype(PEN_)::value && MODE == kLongAll;
    for (int k0 = 0; k0 < Kw; k0 += kLD) {
#pragma unroll
        for (int i = 0; i < kLD; ++i) {
            const int k = k0 + i;
            const f4v x = fixc(buf[i], k);
            buf[i] = ld(k + kLD);
            if (k < Kw) {
                f4v xm = x;
                uint32_t nb = 0u;
                double yv[4] = {0.0, 0.0, 0.0, 0.0};
                if constexpr (PENS) {
                    nb = pnib(NIS_LIDX(k));
                    if (nb) {
                        f4v xp = x;  // the plain elements
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            if ((nb >> q) & 1u) {
                                yv[q] = pen_value(elem(x, q), penf);
                                mex = fmax(mex, yv[q]);
                            }
                        }
                        xm = f4v{(nb & 1u) ? pen_f32_up(yv[0]) : x.x, (nb & 2u) ? pen_f32_up(yv[1]) : x.y,
                                 (nb & 4u) ? pen_f32_up(yv[2]) : x.z, (nb & 8u) ? pen_f32_up(yv[3]) : x.w};
                        xp = f4v{(nb & 1u) ? -INFINITY : x.x, (nb & 2u) ? -INFINITY : x.y,
                                 (nb & 4u) ? -INFINITY : x.z, (nb & 8u) ? -INFINITY : x.w};
                        mex = fmax(mex, (double)r_max4(xp));
                    } else {
                        mex = fmax(mex, (double)r_max4(x));
                    }
                }
                const float m4 = r_max4(xm);
                mx = fmaxf(mx, m4);
                if (__ballot(m4 * chi > Rz + 1.0f)) {
                    const float Rn = ceilf(wmax_f32(mx) * chi);
                    if (fabsf(Rn) < 1e30f) {
                        z = ldexp(z, (int)(Rz - Rn));
                        Rz = Rn;
                    }
                }
                float e0 = r_mass(x.x, czh, czl, Rz), e1 = r_mass(x.y, czh, czl, Rz);
                float e2 = r_mass(x.z, czh, czl, Rz), e3 = r_mass(x.w, czh, czl, Rz);
                if constexpr (PENS) {
                    if (nb) {
                        if (nb & 1u) e0 = (float)pen_mass(yv[0] * c64, Rz);
                        if (nb & 2u) e1 = (float)pen_mass(yv[1] * c64, Rz);
                        if (nb & 4u) e2 = (float)pen_mass(yv[2] * c64, Rz);
                        if (nb & 8u) e3 = (float)pen_mass(yv[3] * c64, Rz);
                    }
                }
                z += (double)((e0 + e1) + (e2 + e3));
                if (MODE == kLongAll && a.stats)
                    nfin += (uint32_t)(x.x > -INFINITY) + (uint32_t)(x.y > -INFINITY) +
                            (uint32_t)(x.z > -INFINITY) + (uint32_t)(x.w > -INFINITY);
                if constexpr (MODE == kLongTopP) {
                    const int Rs = (int)Rz + 24;
#define NIS_LHIST(xq, eq)                                                                      \
                    {                                                                          \
                        const int j_ = d_flr(d_vmax((xq) * chi64, tflo));                      \
                        const uint32_t fm_ = (uint32_t)__builtin_amdgcn_ldexpf((eq), Rs - (j_ >> 6)); \
                        __hip_atomic_fetch_add(&sh.ring[j_ & (kLRing - 1)], (1ull << 48) | fm_, \
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); \
                    }
                    NIS_LHIST(x.x, e0)
                    NIS_LHIST(x.y, e1)
                    NIS_LHIST(x.z, e2)
                    NIS_LHIST(x.w, e3)
#undef NIS_LHIST
                }
            }
        }
    }
    };
    if constexpr (MODE == kLongAll) {
        if (pen) sstream(std::true_type{});
        else sstream(std::false_type{});
    } else {
        sstream(std::false_type{});
    }
    NIS_DTS(1);
    mx = wmax_f32(mx);
    if constexpr (MODE == kLongAll) {
        // the wave's exact max (statistics): with a penalty, of the plain
        // logits and the penalised f64 values
        double me = pen ? mex : (double)mx;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) me = fmax(me, __shfl_xor(me, o));
        if (l == 0) sh.gx[w] = me;
    }
    {
        const uint32_t nan_seen = (uint32_t)(__ballot(z != z) != 0ull);
        const double zw = wsum_f64(z);
        const uint32_t nf = (MODE == kLongAll && a.stats) ? wsum_u32(nfin) : 0u;
        if (l == 0) {
            sh.rec[w] = DRec{mx, Rz, Rw0, nan_seen | (Kw > 0 ? 2u : 0u)};
            sh.tw[w] = zw;  // top-p off: the wave's total (2^R_z units)
            sh.nfin[w] = nf;
        }
    }
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
    // ---- B1 ---------------------------------------------------------------------
    lds_barrier();
    NIS_DTS(2);
    const bool rv = l < kLW;
    const DRec rr = sh.rec[rv ? l : 0];
    const bool has = rv && (rr.flags & 2u);
    const float M = wmax_f32(has ? rr.mx : -INFINITY);
    const float R = (M > -INFINITY && fabsf(M * chi) < 1e30f) ? ceilf(M * chi) : 0.0f;
    const int Ri = (int)R;
    {
        const bool anynan = __ballot(rv && (rr.flags & 1u)) != 0ull;
        const float rw0min = -wmax_f32(has ? -rr.rw0 : -INFINITY);
        // a wave whose first chunk held nothing above -inf keeps reference 0,
        // which may lie far above the wave's values: its fold floor must not
        // lie above R's searched octaves (every wave holding data has its
        // first reference at or below R), and a final reference more than 8
        // octaves above the wave's max costs its masses precision (their f32
        // arguments' rounding grows with depth: 8 octaves, 3e-7) or, past 64
        // octaves, the masses themselves: harmless only for a wave whose max
        // lies 20 or more octaves below R
        const bool hasd = has && rr.mx > -INFINITY;
        const float rw0hi = wmax_f32(hasd ? rr.rw0 : -INFINITY);
        const float cw = ceilf(rr.mx * chi);
        // (with raised first references a wave lying 64 or more octaves below
        // its reference lies as far below R: its masses are 2^-64 of the max)
        const bool gapbad = hasd & (rr.rz - cw > 8.0f) &
                            ((R - cw < 20.0f) | ((rfloor == -INFINITY) & (rr.rz - cw > 64.0f)));
        const bool fin = (M > -INFINITY) & (M < INFINITY) & !anynan & (fabsf(M * chi) < 4096.0f) &
                         (__ballot(gapbad) == 0ull) & (MODE != kLongTopP || (rw0hi <= R));
        if (!fin) return NIS_REJECT_NONFINITE;
        if (MODE == kLongTopP && !(R - rw0min < (float)kLSpan)) {
            if (rnext != nullptr && rfloor == -INFINITY) {
                *rnext = R - (float)(kLSpan - 1);
                return kLSpanRetry;
            }
            return NIS_REJECT_NONFINITE;
        }
    }

    // the walk's last step: the drawn element of float4 x4 (row index i0 of
    // element 0, per-element masses ev in the units of r_run), and the row's
    // result
    double Mst = (double)M;  // the row max for the statistics (top-p off: exact, f64)
    double vfin[4] = {0.0, 0.0, 0.0, 0.0};  // top-p off: the final float4's values (penalised in f64)
    auto finish = [&](const f4v& x4, uint32_t i0, const float ev[4], double r_run, double Zk,
                      double Zall, uint64_t kept) {
        int q = -1, qlast = 0;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            if (ev[qq] > 0.0f) {
                qlast = qq;
                if (q < 0) {
                    r_run -= (double)ev[qq];
                    if (r_run <= 0.0) q = qq;
                }
            }
        }
        if (q < 0) q = qlast;
        const double u = sh.u0;
        const double xq = (MODE == kLongAll) ? vfin[q] : (double)elem(x4, q);
        uint32_t tok = i0 + (uint32_t)q;
        if (u == 0.0) tok = 0u;  // r == 0 stops the reference's walk at index 0
        emit_token(a, row, tok);
        if (a.stats) {
            const double rho = exp2((double)R - Mst * c64);  // 2^R units -> max-element units
            const double em = exp2(xq * c64 - Mst * c64);
            write_row_stats(a, row, tok, NIS_PATH_DRAW, Mst / temp, Zk * rho, Zall * rho, u,
                            (u == 0.0) ? 0.0 : em / (Zk * rho), kept, 1, prior);
        }
    };

    // =====================================================================
    if constexpr (MODE == kLongAll) {
        // ---- top-p off: every element kept ----------------------------------
        // (each wave's total rescaled exactly in f64, however far below R the
        // wave lies: one ~1075 octaves down holds 0, as exp(w - max) does in
        // the reference's f64)
        const double T = rv ? ldexp(sh.tw[l], (int)(rr.rz - R)) : 0.0;  // 2^R units
        const double Tincl = rscan16_f64(T);
        const double Z = bcast_f64(Tincl, 15);
        if (!(Z > 0.0) || !(Z < INFINITY)) return NIS_REJECT_NONFINITE;
        if (w == 0 && l < 4) a.rng[4 * (int64_t)row + l] = rst;
        const double r = sh.u0 * Z;
        const uint64_t hw = __ballot(rv & (T > 0.0) & (Tincl >= r));
        const uint64_t nzw = __ballot(rv & (T > 0.0));
        const int ws = hw ? (__ffsll((long long)hw) - 1) : (63 - __clzll((long long)(nzw | 1ull)));
        if (w != ws) return NIS_REJECT_NONE;
        {
            double me = rv ? sh.gx[l] : -INFINITY;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) me = fmax(me, __shfl_xor(me, o));
            Mst = me;
        }
        // a float4's masses (2^R_z units) and values as the stream took them
        auto wmass4 = [&](const f4v& x, int k, float ev[4], double vv[4]) {
            ev[0] = r_mass(x.x, czh, czl, Rz);
            ev[1] = r_mass(x.y, czh, czl, Rz);
            ev[2] = r_mass(x.z, czh, czl, Rz);
            ev[3] = r_mass(x.w, czh, czl, Rz);
#pragma unroll
            for (int q = 0; q < 4; ++q) vv[q] = (double)elem(x, q);
            if (pen) {
                const uint32_t nb = pnib(NIS_LIDX(k));
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if ((nb >> q) & 1u) {
                        vv[q] = pen_value(elem(x, q), penf);
                        ev[q] = (float)pen_mass(vv[q] * c64, Rz);
                    }
                }
            }
        };
        double rk = ldexp(r - bcast_f64(Tincl - T, ws), (int)(R - Rz));  // 2^R_z units
        // this wave's chunks in order until the one holding the crossing (the
        // last with mass if rounding leaves r above every prefix)
        int kc = -1, klast = 0;
        for (int k = 0; k < Kw && kc < 0; ++k) {
            const f4v x = fixc(ld(k), k);
            float e4[4];
            double v4[4];
            wmass4(x, k, e4, v4);
            const float s4 = (e4[0] + e4[1]) + (e4[2] + e4[3]);
            const double ct = wsum_f64((double)s4);
            if (ct > 0.0) {
                klast = k;
                if (ct >= rk) kc = k;
                else rk -= ct;
            }
        }
        if (kc < 0) kc = klast;
        const f4v xc = fixc(ld(kc), kc);
        float ev[4];
        wmass4(xc, kc, ev, vfin);
        const double sl = (double)((ev[0] + ev[1]) + (ev[2] + ev[3]));
        const double lincl = wscan_f64(sl);
        const uint64_t hl = __ballot((sl > 0.0) & (lincl >= rk));
        const uint64_t nzl = __ballot(sl > 0.0);
        const int lc = hl ? (__ffsll((long long)hl) - 1) : (63 - __clzll((long long)(nzl | 1ull)));
        const uint32_t nkept = a.stats ? wsum_u32(l < kLW ? sh.nfin[l] : 0u) : 0u;
        if (l == lc) finish(xc, (uint32_t)NIS_LIDX(kc), ev, rk - (lincl - sl), Z, 0.0, (uint64_t)nkept);
        return NIS_REJECT_NONE;
    }

    // =====================================================================
    // ---- top-p: cutoff search over the 32 octaves below R ----------------
    const float p = a.top_p;
    const int jt0 = 64 * Ri - 64 * kLQ * w - kLQ * l;  // lane: buckets jt0 .. jt0 - kLQ + 1
    unsigned long long bm[kLQ];
    uint32_t bc[kLQ];
#pragma unroll
    for (int q = 0; q < kLQ; ++q) {
        const int j = jt0 - q;
        const unsigned long long v = sh.ring[j & (kLRing - 1)];
        bc[q] = (uint32_t)(v >> 48);
        bm[q] = d_u44(v, j >> 6, Ri);
    }
    unsigned long long lm = 0ull;
    uint32_t lcn = 0u;
#pragma unroll
    for (int q = 0; q < kLQ; ++q) {
        lm += bm[q];
        lcn += bc[q];
    }
    const unsigned long long im = rscan_u64w(lm);
    const uint32_t ic = wscan_u32(lcn);
    // the 32 octaves below the search (and the folded bucket) still count in Z
    unsigned long long lo = 0ull;
#pragma unroll
    for (int q = 0; q < kLQ; ++q) {
        const int j = jt0 - q - 64 * kLSpan;
        lo += d_u44(sh.ring[j & (kLRing - 1)], j >> 6, Ri);
    }
    lo = wsum_u64(lo);
    if (l == 63) {
        sh.wtm[w] = im;
        sh.wtc[w] = ic;
        sh.wlo[w] = lo;
    }
    lds_barrier();  // B2
    const unsigned long long wmi = rscan16_u64(rv ? sh.wtm[l] : 0ull);
    const uint32_t wci = rscan_u32(rv ? sh.wtc[l] : 0u);
    const unsigned long long wli = rscan16_u64(rv ? sh.wlo[l] : 0ull);
    // Z in 2^(R - 44) units
    const unsigned long long Z = rbcast_u64(wmi, kLW - 1) + rbcast_u64(wli, kLW - 1);
    const double pz = (double)p * (double)Z;
    {
        unsigned long long G = (w > 0 ? rbcast_u64(wmi, w - 1) : 0ull) + (im - lm);
        uint32_t C = (w > 0 ? bcast_u32(wci, w - 1) : 0u) + (ic - lcn);
        int jp = INT32_MAX;
        unsigned long long gp_ = 0ull;
        uint32_t np_ = 0u, cp_ = 0u;
#pragma unroll
        for (int q = 0; q < kLQ; ++q) {
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
        const int Lp = pm ? 63 - __clzll((long long)pm) : 0;
        if (l == Lp) sh.cand[w] = DCand{gp_, jp, np_, cp_, 0u};
    }
    lds_barrier();  // B3
    NIS_DTS(3);
    const DCand cd = sh.cand[rv ? l : 0];
    const uint32_t ckey = rv ? ((uint32_t)cd.j ^ 0x80000000u) : 0xFFFFFFFFu;
    const uint32_t kbest = wmin_u32(ckey);
    if (kbest == ((uint32_t)INT32_MAX ^ 0x80000000u)) return NIS_REJECT_WINDOW;
    const int Lb = __ffsll((long long)__ballot(rv && ckey == kbest)) - 1;
    const int bp = (int)(kbest ^ 0x80000000u);
    // every element below the searched range must be removed: even the
    // largest possible one (the range's floor) fails the rule
    if (!((double)Z - d_mup(64 * Ri - 64 * kLSpan, 0, Ri) > pz)) return NIS_REJECT_WINDOW;
    const unsigned long long Gp = rbcast_u64(cd.g, Lb);
    const uint32_t nsel0 = bcast_u32(cd.n, Lb);
    const uint32_t nab0 = bcast_u32(cd.nab, Lb);

    // ---- the cutoff bucket's members -------------------------------------------
    int lv = 0, B = bp;
    unsigned long long Gc = Gp;
    uint32_t ns = nsel0, nabv = nab0;
    float chiL = chi64;
    bool all_out = false;  // no sub-bucket passes: the whole bucket is removed
    // One refinement step of the cutoff bucket (lv, B): add(o, chiL, chiS)
    // puts its members into the 64 sub-buckets of the next level; wave 0
    // takes the deepest passing one (G(s) - m_up(s) <= p Z), every wave reads
    // the result.  Returns false when no sub-bucket passes.
    auto refine = [&](auto&& add) -> bool {
        const int o = B >> (6 * (lv + 1));
        add(o, chiL, chiL * 64.0f);
        lds_barrier();
        if (w == 0) {
            const unsigned long long v = sh.sub[63 - l];  // lane l: sub-bucket 63 - l
            const uint32_t n = (uint32_t)(v >> 48);
            const unsigned long long m = d_u44(v, o, Ri);
            const unsigned long long Gs = Gc + (rscan_u64w(m) - m);
            const uint32_t Cs = nabv + (wscan_u32(n) - n);
            const int Fs = 64 * B + 63 - l;
            const uint64_t ps = __ballot((n != 0u) && ((double)Gs - d_mup(Fs, lv + 1, Ri) <= pz));
            DCut c;
            c.kcut = ~0ull;
            c.nkept = 0u;
            c.rej = ps ? 0u : 1u;
            const int Ls = ps ? 63 - __clzll((long long)ps) : 0;
            c.bj = ps ? 64 * B + 63 - Ls : B;
            c.lv = ps ? lv + 1 : lv;
            c.g = ps ? rbcast_u64(Gs, Ls) : Gc;
            c.nsel = ps ? bcast_u32(n, Ls) : 0u;
            c.nab = ps ? bcast_u32(Cs, Ls) : nabv;
            sh.sub[l] = 0ull;  // (lane 63 - l read it above) cleared for the next level
            if (l == 0) sh.cut = c;
        }
        lds_barrier();
        const DCut c = sh.cut;
        B = c.bj;
        lv = c.lv;
        Gc = c.g;
        ns = c.nsel;
        nabv = c.nab;
        if (c.rej) return false;
        chiL *= 64.0f;
        return true;
    };
    auto sub_add = [&](float x, int o, float cl, float cs, bool valid) {
        const bool mem = valid & (d_flr(x * cl) == B);
        if (__ballot(mem)) {
            const uint32_t fm = r_fm(x, chi, clo, o);
            const uint32_t sb = (uint32_t)d_flr(x * cs) & 63u;
            if (mem)
                __hip_atomic_fetch_add(&sh.sub[sb], (1ull << 48) | (unsigned long long)fm,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    };
    // more members than the list holds: refine by reading the row again
    while (!all_out && ns > (uint32_t)kLMem) {
        if (lv == kDLevels - 1) return NIS_REJECT_CAPACITY;
        all_out = !refine([&](int o, float cl, float cs) {
#pragma unroll
            for (int i = 0; i < kLD; ++i) buf[i] = ld(i);
            for (int k0 = 0; k0 < Kw; k0 += kLD) {
#pragma unroll
                for (int i = 0; i < kLD; ++i) {
                    const int k = k0 + i;
                    const f4v x = fixc(buf[i], k);
                    buf[i] = ld(k + kLD);
#pragma unroll
                    for (int q = 0; q < 4; ++q) sub_add(elem(x, q), o, cl, cs, k < Kw);
                }
            }
        });
    }
    // ---- a second read of the row: the mass of everything above the cutoff
    // bucket (kept whole), and the bucket's members into the list ------------
    double above = 0.0;  // this lane's kept mass above the bucket (2^R_z units)
    {
        const float cl = chiL;
        const int Bt = all_out ? INT32_MIN : B;  // (no members when the bucket is out)
#pragma unroll
        for (int i = 0; i < kLD; ++i) buf[i] = ld(i);
        for (int k0 = 0; k0 < Kw; k0 += kLD) {
#pragma unroll
            for (int i = 0; i < kLD; ++i) {
                const int k = k0 + i;
                const f4v x = fixc(buf[i], k);
                buf[i] = ld(k + kLD);
                if (k < Kw) {
                    float e[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float xq = elem(x, q);
                        const int F = d_flr(xq * cl);
                        e[q] = (F > B) ? r_mass(xq, czh, czl, Rz) : 0.0f;
                        const bool mem = F == Bt;
                        const uint64_t mb = __ballot(mem);
                        if (mb) {
                            uint32_t b0 = 0u;
                            if (l == 0) b0 = atomicAdd(&sh.nmem, (uint32_t)__popcll(mb));
                            const uint32_t sm = bcast_u32(b0, 0) + lane_rank(mb);
                            if (mem && sm < (uint32_t)kLMem)
                                sh.lmem[sm] = LMem{xq, (uint32_t)(NIS_LIDX(k) + q)};
                        }
                    }
                    above += (double)((e[0] + e[1]) + (e[2] + e[3]));
                }
            }
        }
    }
    const double Tabove = wsum_f64(above);
    lds_barrier();
    NIS_DTS(4);
    const uint32_t nml = sh.nmem;  // members listed
    if (!all_out && nml != ns) return NIS_REJECT_BUCKET;
    const int nm = (int)min(nml, (uint32_t)kLMem);
    // refine within the list while more than kDMem remain
    while (!all_out && ns > (uint32_t)kDMem) {
        if (lv == kDLevels - 1) return NIS_REJECT_CAPACITY;
        all_out = !refine([&](int o, float cl, float cs) {
            for (int j = tid; j < nm; j += kLB) sub_add(sh.lmem[j].x, o, cl, cs, true);
        });
    }
    // the final bucket's members (at most kDMem) ranked exactly by wave 0
    if (tid == 0) sh.cnt = 0u;
    lds_barrier();
    if (!all_out && ns > 0u) {
        const int o = B >> (6 * (lv + 1));
        for (int j0 = 0; j0 < nm; j0 += kLB) {
            const int j = j0 + tid;
            const LMem m = sh.lmem[min(j, kLMem - 1)];
            const bool mem = (j < nm) && (d_flr(m.x * chiL) == B);
            const uint64_t mb = __ballot(mem);
            if (mb) {
                uint32_t b0 = 0u;
                if (l == 0) b0 = atomicAdd(&sh.cnt, (uint32_t)__popcll(mb));
                const uint32_t sm = bcast_u32(b0, 0) + lane_rank(mb);
                if (mem) sh.mem[min(sm, (uint32_t)kDMem - 1u)] = RCand{m.x, m.idx, o, r_fm(m.x, chi, clo, o)};
            }
        }
    }
    if (tid < kLW) sh.tmem[tid] = 0.0;
    lds_barrier();
    NIS_DTS(5);
    if (!all_out && sh.cnt != ns) return NIS_REJECT_BUCKET;
    if (w == 0) {
        DCut c;
        c.bj = B;
        c.lv = lv;
        c.g = Gc;
        c.nab = nabv;
        c.nsel = ns;
        c.rej = 0u;
        c.kcut = ~0ull;
        c.nkept = 0u;
        if (!all_out) {
            const int n = (int)ns;
            const bool valid = l < n;
            const RCand mr = sh.mem[min(l, kDMem - 1)];
            const unsigned long long Km = valid ? r_key(mr.x, mr.idx) : 0ull;
            const unsigned long long em = valid ? d_u44(mr.fm, mr.b, Ri) : 0ull;
            unsigned long long pre = 0ull;
            uint32_t rk = 0u;
            for (int j = 0; j < n; ++j) {
                const unsigned long long Kj = rbcast_u64(Km, j);
                const unsigned long long ej = rbcast_u64(em, j);
                pre += (Kj > Km) ? ej : 0ull;
                rk += (Kj > Km) ? 1u : 0u;
            }
            // sampler.rs:150 in rank order
            const bool pass = valid & ((double)(Gc + pre) - (double)em <= pz);
            uint32_t nkept = (uint32_t)n;
            if (__ballot(valid & !pass)) nkept = wmin_u32((valid && !pass) ? rk : 0xFFFFFFFFu);
            const uint64_t lastm = __ballot(valid & (rk + 1u == nkept));
            c.kcut = lastm ? rbcast_u64(Km, __ffsll((long long)lastm) - 1) : ~0ull;
            c.nkept = nkept;
        }
        if (l == 0) sh.cut = c;
    }
    lds_barrier();  // B5: the cutoff is known
    NIS_DTS(6);
    const DCut cut = sh.cut;
    const int Bf = cut.bj;
    const unsigned long long kcut = cut.kcut;
    chiL = chi64;
    for (int i = 0; i < cut.lv; ++i) chiL *= 64.0f;
    // the listed members that are kept join their wave's kept mass
    const int span = 4 * 64 * cpw;  // row indices per wave
    for (int j = tid; j < nm; j += kLB) {
        const LMem m = sh.lmem[j];
        if (d_kept(m.x, m.idx, chiL, Bf, kcut)) {
            const int ow = min((int)((m.idx + (uint32_t)mis) / (uint32_t)span), kLW - 1);
            __hip_atomic_fetch_add(&sh.tmem[ow], (double)r_mass(m.x, czh, czl, sh.rec[ow].rz),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    lds_barrier();
    if (l == 0) sh.tw[w] = ldexp(Tabove + sh.tmem[w], (int)(Rz - R));  // 2^R units (exact)
    if (w == 0 && l < 4) a.rng[4 * (int64_t)row + l] = rst;
    lds_barrier();  // B6
    NIS_DTS(7);
    const double T = rv ? sh.tw[l] : 0.0;
    const double Tincl = rscan16_f64(T);
    const double Zk = bcast_f64(Tincl, 15);
    const double r = sh.u0 * Zk;
    const uint64_t hw = __ballot(rv & (T > 0.0) & (Tincl >= r));
    const uint64_t nzw = __ballot(rv & (T > 0.0));
    const int ws = hw ? (__ffsll((long long)hw) - 1) : (63 - __clzll((long long)(nzw | 1ull)));
    if (w != ws) {
        NIS_DTFLUSH();
        return NIS_REJECT_NONE;
    }
    double rk = ldexp(r - bcast_f64(Tincl - T, ws), (int)(R - Rz));  // 2^R_z units
    // this wave's chunks read again, in order, until the one holding the
    // crossing (the last with kept mass if rounding leaves r above them all)
    int kc = -1, klast = 0;
    f4v xc = ninf4, xlast = ninf4;
    float vc = 0.0f, vlast = 0.0f;
    double rkc = 0.0, rklast = 0.0;
    float evc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, evl[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < kLD; ++i) buf[i] = ld(i);
    for (int k0 = 0; k0 < Kw && kc < 0; k0 += kLD) {
#pragma unroll
        for (int i = 0; i < kLD; ++i) {
            const int k = k0 + i;
            const f4v x = fixc(buf[i], k);
            buf[i] = ld(k + kLD);
            if (k < Kw && kc < 0) {
                float ev[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float xq = elem(x, q);
                    ev[q] = d_kept(xq, (uint32_t)(NIS_LIDX(k) + q), chiL, Bf, kcut) ? r_mass(xq, czh, czl, Rz) : 0.0f;
                }
                const float v = (ev[0] + ev[1]) + (ev[2] + ev[3]);
                const double ct = wsum_f64((double)v);
                if (ct > 0.0) {
                    klast = k;
                    xlast = x;
                    vlast = v;
                    rklast = rk;
#pragma unroll
                    for (int q = 0; q < 4; ++q) evl[q] = ev[q];
                    if (ct >= rk) {
                        kc = k;
                        xc = x;
                        vc = v;
                        rkc = rk;
#pragma unroll
                        for (int q = 0; q < 4; ++q) evc[q] = ev[q];
                    } else {
                        rk -= ct;
                    }
                }
            }
        }
    }
    if (kc < 0) {
        kc = klast;
        xc = xlast;
        vc = vlast;
        rkc = rklast;
#pragma unroll
        for (int q = 0; q < 4; ++q) evc[q] = evl[q];
    }
    NIS_DTS(8);
    {
        const double sl = (double)vc;
        const double lincl = wscan_f64(sl);
        const uint64_t hl = __ballot((sl > 0.0) & (lincl >= rkc));
        const uint64_t nzl = __ballot(sl > 0.0);
        const int lc = hl ? (__ffsll((long long)hl) - 1) : (63 - __clzll((long long)(nzl | 1ull)));
        if (l == lc)
            finish(xc, (uint32_t)NIS_LIDX(kc), evc, rkc - (lincl - sl), Zk, (double)Z / 17592186044416.0,
                   (uint64_t)(cut.nab + cut.nkept));
    }
    NIS_DTS(9);
    NIS_DTFLUSH();
    return NIS_REJECT_NONE;
#undef NIS_LIDX
}

// One 512-lane workgroup per long row (two share a CU, so one's tail runs
// beside the other's stream).  A row the long path declines or cannot take
// gets the token kLPending | reason, and sample_rows_pending_kernel, launched
// after it, runs the general path on exactly those rows.
template <int MODE>
__global__ __launch_bounds__(kLB, 2) void sample_rows_long_kernel(RowArgs a) {
    __shared__ LongShared sh;
    const int row = (int)blockIdx.x;
    if (a.done != nullptr && a.done[row]) return;  // a finished sequence (decode step)
    asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.temperature), "s"(a.top_p),
                 "s"(a.penalty), "s"(a.gen_ids), "s"(a.gen_off));
    uint32_t reject = NIS_REJECT_SHAPE;
    if (long_eligible<MODE>(a, row)) {
        float rn = 0.0f;
        reject = long_row<MODE>(a, row, sh, NIS_REJECT_NONE, -INFINITY, MODE == kLongTopP ? &rn : nullptr);
        if (reject == NIS_REJECT_NONE) return;
        // (|R| < 4096: the retry's floor fits the token's low 14 bits)
        if (reject == kLSpanRetry) reject = kLSpanFlag | ((uint32_t)((int)rn + 8192) & 0x3FFFu);
    }
    if (threadIdx.x == 0) a.tokens[row] = kLPending | reject;
}

// The general path for the rows a long-row launch declined (their token holds
// kLPending | reason).  At most one workgroup per CU, each stepping over the
// rows with the grid's stride, so a launch with nothing pending costs one
// token read per row.
// A top-p row declined for its span alone (kLSpanFlag) runs the long-row
// method once more first, with every first reference raised to the floor
// the token carries.
union PendingShared {
    GeneralShared g;
    LongShared l;
};
__global__ __launch_bounds__(kBlock) void sample_rows_pending_kernel(RowArgs a, int32_t B) {
    __shared__ PendingShared sh;
    for (int row = (int)blockIdx.x; row < B; row += (int)gridDim.x) {
        if (a.done != nullptr && a.done[row]) continue;
        const uint32_t t = a.tokens[row];
        if ((t & kLPending) != kLPending) continue;
        uint32_t reason = t & ~kLPending;
        __syncthreads();  // (every lane has read the marker before a result overwrites it)
        if (reason & kLSpanFlag) {
            const float rfl = (float)((int)(reason & 0x3FFFu) - 8192);
            const uint32_t rj = long_row<kLongTopP>(a, row, sh.l, NIS_REJECT_NONE, rfl, nullptr);
            __syncthreads();  // (every wave has left it before the shared state is used again)
            if (rj == NIS_REJECT_NONE) continue;
            reason = rj;
        }
        general_row<1>(a, row, sh.g, reason);
        __syncthreads();  // (the next row reuses the shared state)
    }
}

}  // namespace nis
