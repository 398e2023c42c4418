// long_sparse_path.h — top-p rows too long for the registers, read once
// (53245 < V <= 262141, 0 < top_p < 0.95, T > 0, no top-k, no penalty
// history; src/sampler.rs:118-160, 201-216).  One row per 1024-lane
// workgroup (16 wave64s); the row's candidates live in LDS.
//
// Layout as in the sparse kernel: wave w owns the contiguous 64-slot chunks
// [cpw w, cpw (w + 1)) of the row's float4 slots, lane l of chunk k holds
// slot 64 (cpw w + k) + l; each lane keeps kLSD nontemporal loads in flight
// in a ring of registers.
//
// Listing threshold.  Chunks 0 and 1 of every wave (8 elements per lane)
// are pooled into one count histogram of x*c on 1/16-octave bins (a ring of
// 64 octaves) behind one barrier; every wave then reads the same threshold
// thl off it: the lower edge of the deepest bin, counted down from the
// sample's max, holding at most a share kLSQ of the sample (less when V is
// so large that the lists could not hold that share).  Every element with
// x c >= thl is listed by its wave (its value, and its place in the chunk as
// one byte; entries before each chunk counted per chunk), in row order, and
// 64 at a time the listed elements join the exact histograms (1/64-octave
// buckets on an absolute grid, count << 48 | octave-relative fixed-point
// mass, and whole octaves in 8 copies) while the stream goes on.  Z is the
// f64 sum of 2^(x c - R0) over every element, R0 = ceil(sample max * c).
//
// After the stream the tail is the sparse kernel's: the complete range is
// x c >= x_lo = max(thl, M c - kLSDeep) (nothing deeper is kept at top-p <
// 0.95: at most V 2^-24 Z <= 0.016 Z lies there), wave 0 finds the cutoff
// bucket b_p by the two-level search, every wave sums its kept masses per
// lane segment of its list and lists its members of b_p, and the last wave
// ranks the members and walks waves -> the chosen wave's segment ->
// elements.  Masses are exact integers in 2^(R - 40) units, as there.
//
// A row this path cannot prove (a list past capacity, a nucleus reaching
// below thl, non-finite values) returns a reject code before anything is
// written; the kernel then runs the long-row method (long_path.h, which
// reads the row again) and, should that decline too, the general path.
#pragma once
#include "sparse_path.h"
#include "long_path.h"

namespace nis {

constexpr int kLSB = 1024;                     // lanes per workgroup
constexpr int kLSW = kLSB / 64;                // waves per workgroup
constexpr int kLSK = 64;                       // float4 chunks per lane (at most)
constexpr int kLSMaxV = kLSB * 4 * kLSK - 3;   // 262141
constexpr int kLSD = 4;                        // loads in flight ahead of the chunk in use
constexpr int kLSR = kLSD + 1;                 // register slots of the load ring
constexpr int kLSE = 1672;                     // listed elements per wave
constexpr int kLSMem = 256;                    // members of the cutoff bucket (ranked by one wave)
constexpr int kLSBins = 1024;                  // sample bins: 1/16 octave, a ring of 64 octaves
constexpr float kLSQ = 0.17f;                  // sampled share at or above thl (at most)
constexpr float kLSFill = 0.82f;               // expected lists at most this share of capacity
// Octaves below the row max past which nothing is kept: V 2^-24 <= 0.016 <
// 0.05 <= 1 - top_p for V <= 262141.
constexpr float kLSDeep = 24.0f;
static_assert(kLSMaxV * 0.000000059604644775390625 < 0.05, "depth bound for this V");

struct LSShared {
    float ent[kLSW][kLSE + 4];          // listed elements, row order per wave (entry kLSE: dump slot)
    uint8_t epos[kLSW][kLSE + 4];       //   their place in the chunk: 4 * lane + element
    uint16_t ccnt[kLSW][kLSK + 2];      // entries listed before chunk k (k = Kw: all of them)
    union alignas(16) {
        unsigned long long hist[kSHB];  // [b & (kSHB-1)]: count << 48 | sum of fm (to the search)
        struct {
            SMem mem[kLSMem];                // members of b_p (after the search)
            uint32_t scnt[64];               // their sub-buckets: count,
            double smass[64];                //   mass (2^(R-40) units),
            unsigned long long smup[64];     //   largest member's mass (f64 bits)
            unsigned long long sk[kLSMem];   // the members of the cutoff sub-bucket: keys,
            double se[kLSMem];               //   masses
        };
    };
    union alignas(16) {
        uint32_t sbin[kLSBins];         // the pooled sample (before the listing)
        double seg[kLSW][64];           // kept mass above b_p per lane segment (after the search)
    } u;
    double tw[kLSW];                    // per-wave kept mass (2^(R-40) units, integers)
    SRec rec[kLSW];
    SCut cut;
    double u0;                          // the draw
    uint32_t nmem;
    uint32_t cnt2;                      // waves done with their kept sums
    uint32_t kmax;                      // max logit (order-preserving key)
    uint32_t ksmp;                      // max of the sample
    uint32_t nmax;                      // largest list
};
static_assert(sizeof(LSShared) <= 163840, "LDS of one workgroup");

// u64 wave minimum by two DPP u32 minima (the high words, then the low
// words of the lanes holding the smallest high word), uniform.
__device__ __forceinline__ unsigned long long wmin_u64(unsigned long long v) {
    const uint32_t hi = wmin_u32((uint32_t)(v >> 32));
    const uint32_t lo = wmin_u32((uint32_t)(v >> 32) == hi ? (uint32_t)v : 0xFFFFFFFFu);
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ bool lsparse_eligible(const RowArgs a, int row) {
    if (a.V <= kSMaxV || a.V > kLSMaxV) return false;
    if (!(a.temperature > 0.0f) || !(a.top_p > 0.0f) || !(a.top_p < 0.95f)) return false;
    if (a.top_k > 0 && a.top_k < (uint64_t)a.V) return false;
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1) && g1 > g0) return false;
    return true;
}

// Returns NIS_REJECT_NONE when the row is done, else (uniformly across the
// workgroup) why it must be recomputed; nothing has been written then.
__device__ __forceinline__ uint32_t lsparse_row(const RowArgs a, const int row, LSShared& sh) {
    const int l = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int V = (int)a.V;
    const gfp rowp = (gfp)(a.logits + (int64_t)row * a.ld);
    const int mis = (int)(((uintptr_t)rowp >> 2) & 3);  // elements before the row in its 16 B block
    const gf4p base = (gf4p)(rowp - mis);
    const int f_lo = mis ? 1 : 0;          // first float4 slot lying fully inside the row
    const int f_hi = (V + mis - 4) >> 2;   // last one
    const int nsl = (V + mis + 3) >> 2;    // slots touching the row
    const int cpw = (((nsl + 63) >> 6) + kLSW - 1) / kLSW;  // chunks per wave (<= kLSK)
    const int wbase = 64 * cpw * w;
    const int Kw = min(max((nsl - wbase + 63) >> 6, 0), cpw);
    const int slot0 = wbase + l;
    const int tid = (int)threadIdx.x;

    // the (at most 3 + 3) elements of partial head / tail slots
    const float hv = rowp[(l < 3) ? l : ((l < 6) ? V - 6 + l : 0)];
    __builtin_amdgcn_sched_barrier(0);
    const uint64_t bptr = (uint64_t)(uintptr_t)base;
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    const int voff = 16 * slot0;
    f4v xv[kLSR];
    xv[0] = nis_buffer_load_f4(rsrc, (Kw > 0) ? 16 * max(slot0, f_lo) : 0x7FFFFFF0, 0, 2);
    __builtin_amdgcn_sched_barrier(0);
    // the shared state cleared, ordered by one barrier before any use (it
    // sits before the other loads, as in the sparse kernel)
    *reinterpret_cast<u4v*>(&sh.hist[2 * tid]) = u4v{0u, 0u, 0u, 0u};
    sh.u.sbin[tid] = 0u;
    if (tid == 0) {
        sh.nmem = 0u;
        sh.cnt2 = 0u;
        sh.kmax = 0u;
        sh.ksmp = 0u;
        sh.nmax = 0u;
    }
    lds_barrier();
#pragma unroll
    for (int k = 1; k < kLSD; ++k) {
        xv[k] = nis_buffer_load_f4(rsrc, (k < Kw) ? voff + 1024 * k : 0x7FFFFFF0, 0, 2);
        __builtin_amdgcn_sched_barrier(0);  // chunk order = issue order
    }
    typedef const __attribute__((address_space(1))) uint64_t* gu64p;
    uint64_t rsv = 0;
    if (w == 0) rsv = ((gu64p)(a.rng + 4 * (int64_t)row))[l & 3];

    __builtin_amdgcn_s_setprio(0);
    if (w >= kLSW / 4) __builtin_amdgcn_s_setprio(1);
    if (w >= kLSW / 2) __builtin_amdgcn_s_setprio(2);
    if (w >= 3 * kLSW / 4) __builtin_amdgcn_s_setprio(3);

    const float h0 = bcast_f32(hv, 0), h1 = bcast_f32(hv, 1), h2 = bcast_f32(hv, 2);
    const float t0 = bcast_f32(hv, 3), t1 = bcast_f32(hv, 4), t2 = bcast_f32(hv, 5);
    const f4v ninf4 = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    // chunk k as loaded -> its values (partial slots fixed, chunks past the
    // wave's read as -inf)
    auto fixc = [&](f4v v, int k) -> f4v {
        if (k >= Kw) return ninf4;
        const int fb0 = wbase + 64 * k;
        if (fb0 < f_lo || fb0 + 63 > f_hi)
            v = fix_slot(v, slot0 + 64 * k, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2);
        return v;
    };

    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const float c = (float)(1.4426950408889634 / temp);     // log2(e) / T
    const float p = a.top_p;

    // ---- the pooled sample: chunks 0 and 1 of every wave -----------------
    xv[0] = fixc(xv[0], 0);
    xv[1] = fixc(xv[1], 1);
    {
        float ms = -INFINITY;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float x = elem(xv[s], q);
                const bool fin = (x > -INFINITY) & (x < INFINITY);
                const float tb = fminf(fmaxf(floorf(x * c * 16.0f), -1.0e9f), 1.0e9f);
                if (fin) atomicAdd(&sh.u.sbin[(uint32_t)(int)tb & (kLSBins - 1)], 1u);
                ms = s_max(ms, x);
            }
        }
        ms = wmax_f32(ms);
        if (l == 0) atomicMax(&sh.ksmp, key32(ms));
    }
    lds_barrier();
    // every wave reads the same threshold: bins bt - j (j = 16 l + i) from the
    // sample max's bin down, the deepest j whose cumulative count stays
    // within the share
    float thl;
    float R0;
    {
        const float M0 = unkey32(sh.ksmp);
        const bool ok = (M0 > -INFINITY) & (fabsf(M0 * c) < 1.0e6f);
        const int bt = ok ? (int)floorf(M0 * c * 16.0f) : 0;
        uint32_t cnt[16];
        uint32_t s = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            cnt[i] = sh.u.sbin[(uint32_t)(bt - 16 * l - i) & (kLSBins - 1)];
            s += cnt[i];
        }
        const uint32_t incl = wscan_u32(s);
        const uint32_t N = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
        const float share = fminf(kLSQ, kLSFill * (float)(kLSW * kLSE) / (float)V);
        const uint32_t Q = (uint32_t)(share * (float)N);
        uint32_t cum = incl - s;
        int jd = -1;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            cum += cnt[i];
            jd = (cum <= Q) ? 16 * l + i : jd;
        }
        const int J = (int)wmax_f32((float)jd);  // (exact: |jd| < 2^24)
        // J < 0: the max's own bin holds more than the share; only what lies
        // above the sample max is listed then (the row is likely declined)
        thl = ok ? (float)(bt - max(J, -1)) * 0.0625f : INFINITY;
        R0 = ok ? ceilf(M0 * c) : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    // thl in logit units, rounded down (x >= thx whenever x c >= thl), and
    // never below the lowest finite value (-inf is never listed)
    const float thx = thl < INFINITY ? fmaxf(thl / c - fabsf(thl / c) * 1.0e-6f - 1.0e-30f, -3.0e38f)
                                     : INFINITY;

    // ---- stream: Z, max, listing, histogram rounds --------------------------
    double z = 0.0;
    float mx = -INFINITY;
    float cz = c, Rz = R0;
    asm volatile("" : "+v"(cz), "+v"(Rz));
    const uint32_t ent0 = lds_addr(&sh.ent[w][0]), pos0 = lds_addr(&sh.epos[w][0]);
    const uint32_t hist0 = lds_addr(&sh.hist[0]);
    uint32_t nw = 0u;  // listed so far (wave-uniform; past kLSE the row is declined)
    uint32_t nh = 0u;  // of them in the histograms
    // 64 listed elements (entries e0 + l for the lanes of am) into the histograms
    auto hadd = [&](float xq, uint64_t am) {
        const float tq = xq * c;
        const int b = s_bucket(tq);
        const uint32_t fm = s_fm(xq, c, tq);
        const unsigned long long hv = (1ull << 48) | (uint64_t)fm;
        if (am == ~0ull) atomicAdd(&sh.hist[(uint32_t)b & (uint32_t)(kSHB - 1)], hv);  // (a full round)
        else lds_add_u64_m(am, hist0 + 8 * ((uint32_t)b & (uint32_t)(kSHB - 1)), hv);
    };
    auto hround = [&](uint32_t e0, uint64_t am) { hadd(sh.ent[w][min(e0 + (uint32_t)l, (uint32_t)kLSE)], am); };
    for (int k0 = 0; k0 < Kw; k0 += kLSR) {
#pragma unroll
        for (int j = 0; j < kLSR; ++j) {
            const int k = k0 + j;
            // the load kLSD chunks ahead, into the slot chunk k - 1 left
            {
                const int kn = k + kLSD;
                xv[(j + kLSD) % kLSR] = nis_buffer_load_f4(rsrc, (kn < Kw) ? voff + 1024 * kn : 0x7FFFFFF0, 0, 2);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (k < Kw) {
                // one histogram round per chunk while 64 listed elements
                // wait: its entry read goes out first and is used after the
                // masses, so the wave does not stall on it
                const bool rnd = (nw - nh >= 64u) & (nh + 64u <= (uint32_t)kLSE);
                float xr = 0.0f;
                if (rnd) xr = sh.ent[w][nh + (uint32_t)l];
                const f4v x = (k < 2) ? xv[j] : fixc(xv[j], k);
                const float e0 = __builtin_amdgcn_exp2f(fmaf(x.x, cz, -Rz));
                const float e1 = __builtin_amdgcn_exp2f(fmaf(x.y, cz, -Rz));
                const float e2 = __builtin_amdgcn_exp2f(fmaf(x.z, cz, -Rz));
                const float e3 = __builtin_amdgcn_exp2f(fmaf(x.w, cz, -Rz));
                z += (double)((e0 + e1) + (e2 + e3));
                mx = s_max(mx, s_max4(x));
                // listing: element q of this lane goes to entry nw + (the
                // entries of lower lanes) + (its own lower elements); entries
                // past kLSE land in the dump slot
                const bool c0 = x.x >= thx, c1 = x.y >= thx, c2 = x.z >= thx, c3 = x.w >= thx;
                const uint64_t m0 = __ballot(c0), m1 = __ballot(c1), m2 = __ballot(c2), m3 = __ballot(c3);
                if (rnd) {
                    hadd(xr, ~0ull);
                    nh += 64u;
                }
                if (m0 | m1 | m2 | m3) {
                    const uint32_t pre = lane_rank(m0) + lane_rank(m1) + lane_rank(m2) + lane_rank(m3);
                    const uint32_t s0 = nw + pre;
                    const uint32_t s1 = s0 + (c0 ? 1u : 0u);
                    const uint32_t s2 = s1 + (c1 ? 1u : 0u);
                    const uint32_t s3 = s2 + (c2 ? 1u : 0u);
                    // (a chunk adds at most 256 entries: the clamp matters
                    // only near the end of the list)
                    const uint32_t lim = (nw + 256u <= (uint32_t)kLSE) ? 0xFFFFFFFFu : (uint32_t)kLSE;
                    const uint32_t d0 = min(s0, lim), d1 = min(s1, lim);
                    const uint32_t d2 = min(s2, lim), d3 = min(s3, lim);
                    const uint32_t pb = 4u * (uint32_t)l;
                    lds_put_f32_u8(m0, ent0 + 4 * d0, x.x, pos0 + d0, pb);
                    lds_put_f32_u8(m1, ent0 + 4 * d1, x.y, pos0 + d1, pb + 1u);
                    lds_put_f32_u8(m2, ent0 + 4 * d2, x.z, pos0 + d2, pb + 2u);
                    lds_put_f32_u8(m3, ent0 + 4 * d3, x.w, pos0 + d3, pb + 3u);
                }
                if (l == 0) sh.ccnt[w][k] = (uint16_t)nw;
                nw += (uint32_t)(__popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3));
            }
        }
    }
    {
        // the rounds still waiting, the last one partial
        const uint32_t ne = min(nw, (uint32_t)kLSE);
        while (nh + 64u <= ne) {
            hround(nh, ~0ull);
            nh += 64u;
        }
        if (nh < ne) hround(nh, __ballot(nh + (uint32_t)l < ne));
        if (l == 0) sh.ccnt[w][Kw] = (uint16_t)nw;
    }

    // ---- stream end -------------------------------------------------------------
    __builtin_amdgcn_s_setprio(0);
    z = wsum_f64(z);
    mx = wmax_f32(mx);
    {
        const uint64_t zb = (uint64_t)__double_as_longlong(z);
        const uint32_t ra = lds_addr(&sh.rec[w]);
        lds_put_b128_m(1ull, ra, u4v{(uint32_t)zb, (uint32_t)(zb >> 32), __float_as_uint(mx),
                                     __float_as_uint(Rz)});
        lds_put_b128_m(1ull, ra + 16, u4v{__float_as_uint(thl), nw, 0u, 0u});
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
    if (l == 0) {
        atomicMax(&sh.kmax, key32(mx));
        atomicMax(&sh.nmax, nw);
    }
    const uint32_t ne = min(nw, (uint32_t)kLSE);
    const int sg = (int)((ne + 63u) >> 6);  // entries per lane segment
    const int e0 = l * sg;                  // the lane's first entry

    // ---- B1: every listed element is in the histograms -------------------------
    lds_barrier();
    // Ring overrun: listed elements more than 31 octaves below the row max
    // (listed against thl before that max was met) alias in the 32-octave
    // ring.  Every wave subtracts its own (exact: integer counts and
    // fixed-point masses); one barrier orders that before the search.  The
    // complete range lies above x_lo >= M c - kLSDeep, so nothing of it goes.
    {
        const float Mr = unkey32(sh.kmax);
        if ((Mr > -INFINITY) & (Mr < INFINITY) & (fabsf(Mr * c) < 1e6f) & (thl < INFINITY)) {
            const int bMr = s_bucket(Mr * c);
            const int blist = (int)floorf(thl * (float)kSRes) - 2;  // at or below every listed bucket
            if (!(bMr - blist < kSHB - kSRes)) {
                for (int i = 0; i < sg; ++i) {
                    const int e = e0 + i;
                    const float xq = sh.ent[w][min(e, kLSE)];
                    const float tq = xq * c;
                    const int b = s_bucket(tq);
                    const uint64_t am = __ballot((e < (int)ne) & (b <= bMr - (kSHB - kSRes)));
                    if (am)
                        lds_add_u64_m(am, hist0 + 8 * ((uint32_t)b & (uint32_t)(kSHB - 1)),
                                      0ull - ((1ull << 48) | (uint64_t)s_fm(xq, c, tq)));
                }
                lds_barrier();
            }
        }
    }
    const int li = min(l, kLSW - 1);
    const bool rv = l < kLSW;
    if (w == 0) {
        __builtin_amdgcn_s_setprio(3);
        const double rz = rv ? sh.rec[li].z : 0.0;
        const float M = unkey32(sh.kmax);
        const float R = (M > -INFINITY && fabsf(M * c) < 1e30f) ? ceilf(M * c) : 0.0f;
        const int Ri = (int)R;
        const uint32_t nmax = sh.nmax;
        const bool fin = (M > -INFINITY) & (M < INFINITY) & (fabsf(M * c) < 1e6f);
        const float xlo = fmaxf(thl, ceilf((M * c - kLSDeep) * 16.0f) * 0.0625f);
        const bool xfin = fin & (xlo < INFINITY) & (xlo <= M * c);
        const int blo = xfin ? (int)(xlo * (float)kSRes) : 0;  // xlo: a multiple of 1/16
        const int bM = xfin ? s_bucket(M * c) : 0;
        const int oM = bM >> kSLog, olo = blo >> kSLog;
        // level-1 reads: octave oM - l for l <= oM - olo, and octave olo's
        // buckets at or above blo
        const int bl = kSRes * olo + l;
        const unsigned long long lv = (bl >= blo && bl <= bM) ? sh.hist[(uint32_t)bl & (kSHB - 1)] : 0ull;
        const int o = oM - l;
        const bool oin = l <= oM - olo;
        // octave o's sum of its 64 buckets (the rows of the ring it spans,
        // read starting at a lane-rotated pair so the lanes' reads spread
        // over the banks)
        unsigned long long ovr = 0ull;
        if (oin && o != olo) {
            const u4v* const oc = reinterpret_cast<const u4v*>(&sh.hist[kSRes * ((uint32_t)o & 31u)]);
#pragma unroll 8
            for (int j = 0; j < kSRes / 2; ++j) {
                const u4v q = oc[(j + l) & (kSRes / 2 - 1)];
                ovr += (((unsigned long long)q.y << 32) | q.x) + (((unsigned long long)q.w << 32) | q.z);
            }
        }
        const double ZR = r16_sum(rv ? ldexp(rz, (int)(Rz - R)) : 0.0);  // exact rescale
        const double pz = (double)p * ZR * kS40;
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
        if (!fin || !(ZR > 0.0) || !(ZR < INFINITY)) {
            cut.reject = NIS_REJECT_NONFINITE;
        } else if (!xfin || nmax > (uint32_t)kLSE || oM - olo > 30) {
            cut.reject = NIS_REJECT_CAPACITY;
        } else {
            // level 1 (octave olo is the deepest lane; its complete part is
            // summed alongside)
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
            const uint64_t P = __ballot(oin & (on != 0u) & (Go - ldexp(1.0001, o + 1 - Ri + 40) <= pz));
            const uint64_t NEo = __ballot(oin & (on != 0u));
            // everything below blo is removed: G(blo - 1) - m_up(blo - 1) > p Z
            const bool lo_ok = (gtot - s_mup(blo - 1, Ri) > pz) & (gtot < 4503599627370496.0);
            if (!P || !lo_ok) {
                cut.reject = NIS_REJECT_WINDOW;
            } else {
                // level 2: lane l takes bucket 64 O + 63 - l of O = Op, the
                // deepest passing octave, then (when Op has no passing bucket)
                // of Oa, the next non-empty octave above it
                const int lp = 63 - __clzll((long long)P);
                const uint64_t up = NEo & ((1ull << lp) - 1ull);
                const int la = up ? 63 - __clzll((long long)up) : -1;
                int Ls = -1, bs = 0;
                double gs = 0.0;
                uint32_t cs = 0u, ns = 0u;
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
                        const uint64_t sel = pass2 == 0 ? __ballot((bn != 0u) & (Gb - s_mup(b, Ri) <= pz))
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
                if (Ls < 0) {
                    cut.reject = NIS_REJECT_WINDOW;
                } else {
                    cut.bp = (int32_t)bcast_u32((uint32_t)bs, Ls);
                    cut.gp = bcast_f64(gs, Ls);
                    cut.nabove = bcast_u32(cs, Ls);
                    cut.bpd = cut.bp;
                    const uint32_t nbp = bcast_u32(ns, Ls);
                    // the kept range stays within 16 octaves of R (exact fixed point)
                    if ((cut.bp >> kSLog) < Ri - 16) cut.reject = NIS_REJECT_WINDOW;
                    else if (nbp > (uint32_t)kLSMem) cut.reject = NIS_REJECT_BUCKET;
                }
            }
        }
        if (l == 0) sh.cut = cut;
        __builtin_amdgcn_s_setprio(0);
    }
    // ---- B2: the cutoff bucket is known ------------------------------------
    lds_barrier();
    const SCut cut = sh.cut;
    if (cut.reject != NIS_REJECT_NONE) return cut.reject;
    if (w == 0 && l < 4) a.rng[4 * (int64_t)row + l] = rst;
    const int bp = cut.bp;
    const float M = cut.M, R = cut.R;
    const int Ri = (int)R;
    {
        // this wave's kept mass above b_p per lane segment (lane l: entries
        // [l sg, l sg + sg)), and its members of b_p; every element of bucket
        // >= b_p >= blo is listed, and its mass (octave >= R - 16) is an exact
        // integer in 2^(R - 40) units (fm shifted by 0..16)
        unsigned long long isum = 0ull;
        for (int i0 = 0; i0 < sg; i0 += 8) {
          float xb[8];  // the next 8 entries, read before any is used
#pragma unroll
          for (int u = 0; u < 8; ++u) xb[u] = sh.ent[w][min(e0 + i0 + u, kLSE)];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int i = i0 + u;
            const int e = e0 + i;
            const bool in = (i < sg) & (e < (int)ne);
            const float x = xb[u];
            const float t = x * c;
            const int b = s_bucket(t);
            const bool above = in & (b > bp);
            const uint32_t fk = (above | (in & (b == bp))) ? s_fm(x, c, t) : 0u;
            isum += above ? ((unsigned long long)fk << ((uint32_t)((b >> kSLog) - Ri + 16) & 63u)) : 0ull;
            if (in & (b == bp)) {
                // a member: its record (value, entry, fm, wave << 16 | lane
                // segment) in the next slot; its row index is looked up only
                // if the ranking needs it
                const uint32_t slot = atomicAdd(&sh.nmem, 1u);
                sh.mem[min(slot, (uint32_t)kLSMem - 1)] =
                    SMem{x, (uint32_t)e, fk, ((uint32_t)w << 16) | (uint32_t)l};
            }
          }
        }
        const double ssum = (double)isum;
        sh.u.seg[w][l] = ssum;
        const double tsum = wsum_f64(ssum);
        if (l == 0) sh.tw[w] = tsum;
    }
    // ---- the last wave to finish its sums ranks the members and walks -------
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    uint32_t done2 = 0u;
    if (l == 0) done2 = atomicAdd(&sh.cnt2, 1u);
    done2 = bcast_u32(done2, 0);
    if (done2 != (uint32_t)(kLSW - 1)) return NIS_REJECT_NONE;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_s_setprio(3);

    const double pz = cut.pz;
    const double gp = cut.gp;
    // The members of b_p (up to kLSMem; lane l holds l, l + 64, ...) in 64
    // sub-buckets of their value keys (sub-bucket 0: the largest values).
    // The cutoff sub-bucket s* is found like b_p: the deepest non-empty one
    // with G(s) - m_up(s) <= p Z, m_up(s) its largest member's mass (every
    // member of the sub-buckets above s* is then kept: the last of them, y,
    // has D(y) <= G(s*) - 2 m(y) < p Z, as m(y) >= m_up(s*) / 2 within one
    // bucket); only the members of s* are ranked exactly.
    const int n = (int)min(sh.nmem, (uint32_t)kLSMem);
    float xq[4];
    uint32_t kq[4], sq[4], lq[4], eq4[4];  // value key, sub-bucket, wave << 16 | segment, entry
    double eq[4];
    uint32_t vlo = 0xFFFFFFFFu, vhi = 0u;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const int m = l + 64 * r4;
        const bool v = m < n;
        const u4v mr = *reinterpret_cast<const u4v*>(&sh.mem[min(m, kLSMem - 1)]);
        xq[r4] = __uint_as_float(mr.x);
        kq[r4] = v ? key32(xq[r4]) : 0u;
        eq[r4] = v ? s_m40(mr.z, (int)floorf(xq[r4] * c), Ri) : 0.0;
        eq4[r4] = mr.y;  // entry number in its wave's list
        lq[r4] = mr.w;   // wave << 16 | lane segment
        if (v) {
            vlo = min(vlo, kq[r4]);
            vhi = max(vhi, kq[r4]);
        }
    }
    vlo = wmin_u32(vlo);
    vhi = ~wmin_u32(~vhi);
    const float fspan = 64.0f / ((float)(vhi - vlo) + 1.0f);
    sh.scnt[l] = 0u;
    sh.smass[l] = 0.0;
    sh.smup[l] = 0ull;
    lds_wave_fence();
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const bool v = l + 64 * r4 < n;
        // (f32: monotone in the key, so every sub-bucket is a range of keys)
        sq[r4] = v ? 63u - min((uint32_t)((float)(kq[r4] - vlo) * fspan), 63u) : 64u;
        const uint64_t vm = __ballot(v);
        if (vm) {
            const uint32_t si = min(sq[r4], 63u);
            if (v) {
                atomicAdd(&sh.scnt[si], 1u);
                atomicMax(&sh.smup[si], (unsigned long long)__double_as_longlong(eq[r4]));
            }
            lds_add_f64_m(vm, lds_addr(&sh.smass[si]), eq[r4]);
        }
    }
    lds_wave_fence();
    uint32_t cstar = 0u;  // members of s*
    int sstar = -1;
    int sabove = -1;      // the next non-empty sub-bucket above s* (all of it kept)
    double Gstar = 0.0;
    {
        const uint32_t cn = sh.scnt[l];
        const double mm = sh.smass[l];
        const double mu = __longlong_as_double((long long)sh.smup[l]);
        const double Gs = gp + (wscan_f64(mm) - mm);
        const uint64_t P = __ballot((cn != 0u) & (Gs - mu <= pz));
        if (P) {
            sstar = 63 - __clzll((long long)P);
            Gstar = bcast_f64(Gs, sstar);
            cstar = bcast_u32(cn, sstar);
            const uint64_t ne_above = __ballot(cn != 0u) & ((1ull << sstar) - 1ull);
            sabove = ne_above ? 63 - __clzll((long long)ne_above) : -1;
        }
    }
    // s*'s members ranked exactly (compacted in LDS, then 64 at a time): the kept ones are a prefix of the stable order, so
    // K >= Kcut keeps exactly them
    unsigned long long Kcs = ~0ull;  // smallest kept key of s*
    if (sstar >= 0) {
        uint32_t nb = 0u;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const bool in = sq[r4] == (uint32_t)sstar;
            const uint64_t im = __ballot(in);
            // the row indices of these members, one member at a time: its
            // chunk is the last one of its wave whose count of earlier
            // entries is at most its entry (lane k reads chunk k's count)
            uint64_t todo = im;
            while (todo) {
                const int ml = __ffsll((long long)todo) - 1;
                todo &= todo - 1ull;
                const int ww = min((int)(bcast_u32(lq[r4], ml) >> 16), kLSW - 1);
                const uint32_t e = bcast_u32(eq4[r4], ml);
                const int kw = min(max((nsl - 64 * cpw * ww + 63) >> 6, 0), cpw);
                const uint32_t cl = (l < kw) ? (uint32_t)sh.ccnt[ww][l] : 0xFFFFFFFFu;
                const int kc = __popcll(__ballot(cl <= e)) - 1;
                const uint32_t pq = sh.epos[ww][min(e, (uint32_t)kLSE)];
                const uint32_t idx = (uint32_t)(4 * (64 * cpw * ww + 64 * kc + (int)(pq >> 2)) + (int)(pq & 3u) - mis);
                if (l == ml) eq4[r4] = idx;
            }
            const uint32_t pos = nb + lane_rank(im);
            if (in) {
                // stable descending order of sampler.rs:140: value, then index
                sh.sk[pos] = ((unsigned long long)kq[r4] << 32) | (uint32_t)~eq4[r4];
                sh.se[pos] = eq[r4];
            }
            nb += (uint32_t)__popcll(im);
        }
        lds_wave_fence();
        for (uint32_t j0 = 0; j0 < cstar; j0 += 64u) {
            const uint32_t j = j0 + (uint32_t)l;
            const bool mine = j < cstar;
            const unsigned long long Kj = sh.sk[min(j, (uint32_t)kLSMem - 1)];
            const double ej = sh.se[min(j, (uint32_t)kLSMem - 1)];
            double pre = 0.0;
            for (uint32_t t = 0; t < cstar; ++t) pre += (sh.sk[t] > Kj) ? sh.se[t] : 0.0;
            const bool kept = mine & (Gstar + pre - ej <= pz);  // sampler.rs:150
            Kcs = min(Kcs, wmin_u64(kept ? Kj : ~0ull));
        }
    }
    // every member's decision: sub-buckets above s* are kept whole, s*'s
    // members from its ranking.  The last kept key Kcut (b_p's elements at
    // or above it are kept) is s*'s smallest kept key, or with none kept
    // there, the smallest value key of the sub-bucket above (every member
    // with that value is kept, whatever its index).
    unsigned long long Kcut = Kcs;
    if (Kcs == ~0ull && sabove >= 0) {
        uint32_t ka = 0xFFFFFFFFu;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) ka = min(ka, sq[r4] == (uint32_t)sabove ? kq[r4] : 0xFFFFFFFFu);
        Kcut = (unsigned long long)wmin_u32(ka) << 32;
    }
    uint32_t nkept = 0u;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const bool v = l + 64 * r4 < n;
        const bool ins = v & ((int)sq[r4] == sstar);
        bool kept = v & ((int)sq[r4] < sstar);
        if (Kcs != ~0ull) {
            // s*: kept iff the full key reaches Kcs (its members' entries
            // were replaced by their row indices above)
            const uint32_t khi = (uint32_t)(Kcs >> 32);
            kept |= ins & (kq[r4] > khi);
            const bool tie = ins & (kq[r4] == khi);
            kept |= tie & ((uint32_t)~eq4[r4] >= (uint32_t)Kcs);
        }
        const uint64_t keptm = __ballot(kept);
        nkept += (uint32_t)__popcll(keptm);
        if (keptm) {
            const int mw = min((int)(lq[r4] >> 16), kLSW - 1), ms = (int)(lq[r4] & 63u);
            lds_add2_f64_m(keptm, lds_addr(&sh.tw[mw]), lds_addr(&sh.u.seg[mw][ms]), eq[r4]);
        }
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
    // the chosen wave's lane segments
    const double Sl = sh.u.seg[ws][l];
    const double Sincl = wscan_f64(Sl);
    const uint64_t hs = __ballot((Sl > 0.0) & (runw + Sincl >= r));
    const int ls = hs ? (__ffsll((long long)hs) - 1) : 0;
    const double runl = bcast_f64(runw + Sincl - Sl, ls);
    // that segment's entries in row order, one per lane
    const uint32_t nes = min(sh.rec[ws].n, (uint32_t)kLSE);
    const int sgs = (int)((nes + 63u) >> 6);
    const int je = ls * sgs + l;
    const bool inseg = (l < sgs) & (je < (int)nes);
    const int jec = inseg ? je : 0;
    const float xe = sh.ent[ws][jec];
    // its row index: its chunk is the last one whose count of earlier
    // entries is at most the entry (lane k reads chunk k's count)
    uint32_t ide;
    {
        const int kws = min(max((nsl - 64 * cpw * ws + 63) >> 6, 0), cpw);
        const uint32_t cl = (l < kws) ? (uint32_t)sh.ccnt[ws][l] : 0xFFFFFFFFu;
        uint32_t kj = 0u;
        for (int j = 0; j < sgs; ++j) {
            const uint32_t kk = (uint32_t)__popcll(__ballot(cl <= (uint32_t)(ls * sgs + j))) - 1u;
            kj = (l == j) ? kk : kj;
        }
        const uint32_t pq = sh.epos[ws][jec];
        ide = (uint32_t)(4 * (64 * cpw * ws + 64 * (int)kj + (int)(pq >> 2)) + (int)(pq & 3u) - mis);
    }
    const float te = xe * c;
    const int be = s_bucket(te);
    const unsigned long long Ke = ((unsigned long long)key32(xe) << 32) | (uint32_t)~ide;
    const bool kje = inseg & ((be > bp) | ((be == bp) & (Ke >= Kcut)));
    const double ee = kje ? s_m40(s_fm(xe, c, te), (int)floorf(te), Ri) : 0.0;
    const double pe_incl = wscan_f64(ee);
    const uint64_t he = __ballot(kje & (runl + pe_incl >= r));
    const int le = he ? (__ffsll((long long)he) - 1) : 0;
    if (l == le) {
        const uint32_t tok = (u == 0.0) ? 0u : ide;  // r == 0 stops the reference's walk at index 0
        emit_token(a, row, tok);
        if (a.stats) {
            const double prob = (u == 0.0) ? 0.0 : ee / zk;
            // 2^(R - M c): units of 2^R -> units of the max element's mass
            const double rho = (double)__builtin_amdgcn_exp2f(-fmaf(M, c, -R));
            write_row_stats(a, row, tok, NIS_PATH_DRAW, (double)M / temp, zk / kS40 * rho,
                            cut.zr * rho, u, prob, (uint64_t)(cut.nabove + nkept), 1);
        }
    }
    return NIS_REJECT_NONE;
}

}  // namespace nis
