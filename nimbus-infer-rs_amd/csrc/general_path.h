// general_path.h — the general per-row sampler: one 512-lane workgroup per
// row, any V <= NIS_MAX_V, repetition penalty, top-k, top-p and every
// special case of sample() (src/sampler.rs:163-217).  It makes several
// passes over the row (the first from HBM, the others mostly from L2 /
// MALL), each with kGU loads in flight per lane, and is used for the rows
// the register-resident fast path does not take (penalty, top-k, non-finite
// input, V above its capacity) or hands on.
//
// Masses: without a penalty a row's masses are 2^(x*c - R) (c = log2(e)/T
// split as c_hi + c_lo, R = ceil(M*c_hi)), evaluated octave by octave: with
// o = floor(x*c_hi), f32 exp2 of the small argument x*c_lo + (x*c_hi - o),
// scaled by 2^(o - R) in f64.  The argument's rounding then costs 2^-24 of
// an octave at any depth below the max (relative error ~1.6e-7 with exp2's
// own), where one f32 argument x*c - R would lose 2^-24 of its depth.  With
// a penalty the f64 value w = v/T gives 2^((w - M/T) * log2 e), evaluated as
// an f32 exp2 of the leading part times a first-order correction for the
// rest (relative error ~1e-7).  Sums are f64; histogram masses are 2^-40
// fixed point (exact and order-independent).
//
// Sort-free top-p (sampler.rs:118-160): the reference keeps sorted position
// pos iff D(pos) = cum_excl(pos) - q(pos) <= p (normalised).  D is
// non-decreasing in pos, so the kept set is a prefix of the stable order.
// A most-significant-digit radix walk over order-preserving keys carries
// G = mass strictly above the current key range and picks, per digit, the
// last bucket whose first (largest-key) element is kept: G - e_first <= p*Z.
// At the last digit the bucket is one key value K*, i.e. a tie group whose
// members are kept in ascending index order while G + (j-1)*e* <= p*Z.
//
// The inverse-CDF walk (sampler.rs:209-216) runs over chunks of kGChunk
// consecutive elements: their kept masses, a prefix over the chunks, and one
// wave's scan of the chunk holding the crossing.
#pragma once
#include <math.h>

#include "device_common.h"
#include "nimbus_sampler.h"
#include "rng.h"

namespace nis {

struct RowArgs {
    const float* logits;
    int64_t ld;
    int64_t V;
    float temperature;
    float top_p;
    float penalty;
    uint64_t top_k;
    uint64_t* rng;
    const uint32_t* gen_ids;
    const int64_t* gen_off;     // CSR history: row b's ids are gen_ids[gen_off[b] .. gen_off[b+1])
    int32_t* gen_len;           // or, when set, row b's are gen_ids[b cap .. b cap + gen_len[b])
    int64_t gen_cap;
    // decode step (all NULL otherwise): rows with done[b] != 0 are skipped; a
    // row's token joins its history, and a stop id or the budget max_new[b]
    // ends the row
    uint8_t* done;
    uint32_t* gen_out;          // the same history, written
    const int32_t* max_new;
    const uint32_t* stop;
    int32_t n_stop;
    uint32_t* tokens;
    nis_row_stats* stats;
};

// Row b's repetition-penalty history [g0, g1) in gen_ids; false without one.
__device__ __forceinline__ bool gen_range(const RowArgs& a, int row, int64_t& g0, int64_t& g1) {
    if (a.gen_ids == nullptr) return false;
    if (a.gen_len != nullptr) {
        g0 = (int64_t)row * a.gen_cap;
        g1 = g0 + min((int64_t)max(a.gen_len[row], 0), a.gen_cap);
        return true;
    }
    if (a.gen_off == nullptr) return false;
    g0 = a.gen_off[row];
    g1 = a.gen_off[row + 1];
    return true;
}

constexpr int kGU = 16;                          // loads per lane per block of a pass
constexpr int kGChunk = 512;                     // walk chunk: 8 rows of 64 elements
constexpr int kGMaxChunks = NIS_MAX_V / kGChunk;
constexpr double kGFix = 1099511627776.0;        // 2^40 fixed-point mass scale
// SIMPLE top-p: value histogram of t = x*c - R (bin b holds t in
// (-(b+1)/kGVRes, -b/kGVRes], the last bin everything lower) and the
// lane-private lists of the members of the (at most two) bins that can hold
// the cutoff
constexpr int kGVBins = 2048;
constexpr float kGVRes = 32.0f;
constexpr int kGLane = 16;                       // list entries per lane

struct GeneralShared {
    union {
        uint32_t bitmap[NIS_MAX_V / 32];  // penalised-id set of the row
        struct {
            uint32_t cnt[kGVBins];
            unsigned long long mass[kGVBins];  // 2^-40 fixed point
            float lx[kGLane][kBlock];          // [slot][thread]
            uint32_t li[kGLane][kBlock];
        } v;
    } u;
    uint32_t hcnt[256];
    unsigned long long hmass[256];    // 2^-40 fixed point
    unsigned long long hkey[256];
    unsigned long long csum[kGMaxChunks];  // kept mass of each walk chunk (2^-40 fixed point)
    uint32_t tcnt[kGMaxChunks];       // tie-group members before each walk chunk
    double dscr[kWaves];
    uint64_t uscr[kWaves];
    int64_t iscr[kWaves];
    double bd[4];
    int64_t bi[4];
};

// The row's token (one lane per row).  In a decode step it also joins the
// row's history, which ends the row on a stop id, on its budget or when full
// (engine.rs:281-287); the penalty read that history before this point.
__device__ __forceinline__ void emit_token(const RowArgs& a, int row, uint32_t token) {
    a.tokens[row] = token;
    if (a.max_new != nullptr) {
        int64_t n = max(a.gen_len[row], 0);
        if (n < a.gen_cap) a.gen_out[(int64_t)row * a.gen_cap + n] = token;
        n = min(n + 1, a.gen_cap);
        a.gen_len[row] = (int32_t)n;
        bool hit = false;
        for (int s = 0; s < a.n_stop; ++s) hit |= a.stop[s] == token;
        if (hit || n >= (int64_t)a.max_new[row] || n >= a.gen_cap) a.done[row] = 1u;
    }
}

__device__ __forceinline__ void write_row_stats(const RowArgs a, int row, uint32_t token,
                                                uint32_t path, double max_w, double z_kept,
                                                double z_all, double u, double prob,
                                                uint64_t kept, uint32_t kernel,
                                                uint32_t reject = NIS_REJECT_NONE) {
    if (a.stats) {
        nis_row_stats s;
        s.max_w = max_w;
        s.z_kept = z_kept;
        s.z_all = z_all;
        s.u = u;
        s.prob = prob;
        s.kept = kept;
        s.path = path;
        s.token = token;
        s.kernel = kernel;
        s.reject = reject;
        a.stats[row] = s;
    }
}

__device__ __forceinline__ void write_row_result(const RowArgs a, int row, uint32_t token,
                                                 uint32_t path, double max_w, double z_kept,
                                                 double z_all, double u, double prob,
                                                 uint64_t kept, uint32_t kernel,
                                                 uint32_t reject = NIS_REJECT_NONE) {
    emit_token(a, row, token);
    write_row_stats(a, row, token, path, max_w, z_kept, z_all, u, prob, kept, kernel, reject);
}

// Digit range of a most-significant-digit radix walk: bits above `hi_shift+8`
// and below `lo_shift` are common to every candidate key (derived from the
// OR of key ^ key_ref over the candidates).
struct DigitRange {
    int hi_shift;  // shift of the first digit
    int lo_shift;  // shift of the last digit
    bool all_equal;
};
__device__ __forceinline__ DigitRange digit_range(uint64_t diff) {
    DigitRange r;
    r.all_equal = (diff == 0);
    if (r.all_equal) {
        r.hi_shift = r.lo_shift = 0;
        return r;
    }
    const int hb = 63 - __clzll((long long)diff);
    const int lb = __ffsll((long long)diff) - 1;
    r.hi_shift = (hb / 8) * 8;
    r.lo_shift = (lb / 8) * 8;
    return r;
}
__device__ __forceinline__ bool in_prefix(uint64_t key, int shift, uint64_t prefix) {
    return (shift + 8 >= 64) ? true : ((key >> (shift + 8)) == prefix);
}

// Every element j of the row with its raw logit xr (element order within a
// lane is ascending j).  Whole blocks of kGU loads per lane, the next
// block's loads issued before the current one is processed (its indices
// clamped into the row, so the last prefetch stays in bounds), then the
// partial last block with a bounds test.
#define NIS_G_EACH(BODY)                                                          \
    {                                                                             \
        const int64_t gstep_ = (int64_t)kBlock * kGU;                             \
        const int64_t gfull_ = (V / gstep_) * gstep_;                             \
        float xs_[kGU], xn_[kGU];                                                 \
        if (gfull_ > 0) {                                                         \
            _Pragma("unroll") for (int u_ = 0; u_ < kGU; ++u_) xs_[u_] =          \
                x[tid + (int64_t)u_ * kBlock];                                    \
        }                                                                         \
        for (int64_t jb_ = tid; jb_ < gfull_; jb_ += gstep_) {                    \
            _Pragma("unroll") for (int u_ = 0; u_ < kGU; ++u_) xn_[u_] =          \
                x[min(jb_ + gstep_ + (int64_t)u_ * kBlock, V - 1)];               \
            _Pragma("unroll") for (int u_ = 0; u_ < kGU; ++u_) {                  \
                const int64_t j = jb_ + (int64_t)u_ * kBlock;                     \
                const float xr = xs_[u_];                                         \
                BODY                                                              \
            }                                                                     \
            _Pragma("unroll") for (int u_ = 0; u_ < kGU; ++u_) xs_[u_] = xn_[u_];  \
        }                                                                         \
        for (int64_t j = gfull_ + tid; j < V; j += kBlock) {                      \
            const float xr = x[j];                                                \
            BODY                                                                  \
        }                                                                         \
    }

// Wave 0, top-p radix step: the digit buckets d = 255 .. 0 (descending key)
// with count, fixed-point mass and largest key; G0 = mass above them.
// Returns (uniform across the wave) the lowest bucket whose largest element
// is kept (sampler.rs:150: G(d) - e_first(d) <= pZ; qualifying buckets form
// a prefix from the top), the mass above it and its count.
template <typename MassOfKey>
__device__ __forceinline__ void topp_digit_select(const GeneralShared& sh, double G0, double pZ,
                                                  MassOfKey mass_of_key, int* sel, double* gsel,
                                                  uint32_t* nsel) {
    const int l = lane_id();
    // lane l owns buckets 4l .. 4l+3 (ascending key)
    uint32_t cnt[4];
    unsigned long long fm[4], km[4];
    unsigned long long ltot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        cnt[i] = sh.hcnt[4 * l + i];
        fm[i] = sh.hmass[4 * l + i];
        km[i] = sh.hkey[4 * l + i];
        ltot += fm[i];
    }
    // mass of the buckets of higher lanes (exact: integer sums below 2^53)
    const double lt = (double)ltot;
    const double incl = wscan_f64(lt);
    const double tot = bcast_f64(incl, 63);
    double above = tot - incl;  // fixed point
    int low = 256;
    double glow = 0.0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
        const double G = G0 + above / kGFix;
        const bool q = (cnt[i] != 0) && (G - mass_of_key(km[i]) <= pZ);
        low = q ? (4 * l + i) : low;
        glow = q ? G : glow;
        above += (double)fm[i];
    }
    const int best = (int)(-wmax_f32(-(float)low));  // DPP minimum (exact in float)
    const uint64_t own = __ballot(low == best);
    const int owner = own ? (__ffsll((long long)own) - 1) : 0;
    *sel = best;
    *gsel = bcast_f64(glow, owner);
    *nsel = (best < 256) ? sh.hcnt[best] : 0u;
}

// `reject` is recorded in the row's stats: why the fast path declined it.
// SIMPLE: a row without a penalty whose masses have a finite f32 reference;
// the SIMPLE form returns false, having written nothing, for any other row.
// TAG only separates the copies called from kernels of different workgroup
// sizes, so each is compiled for its own register budget.
template <bool SIMPLE, int TAG>
__device__ __noinline__ bool general_row_t(const RowArgs a, const int row, GeneralShared& sh,
                                           const uint32_t reject) {
    const int tid = threadIdx.x, l = lane_id(), w = wave_id();
    const float* __restrict__ x = a.logits + (int64_t)row * a.ld;
    const int64_t V = a.V;

    // ---- repetition penalty set (sampler.rs:83-101) --------------------
    bool pen = false;
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1)) {
        if (SIMPLE && g1 > g0) return false;
        if (!SIMPLE && g1 > g0) {
            pen = true;
            const int64_t nw = (V + 31) >> 5;
            for (int64_t i = tid; i < nw; i += kBlock) sh.u.bitmap[i] = 0u;
            __syncthreads();
            for (int64_t i = g0 + tid; i < g1; i += kBlock) {
                const uint32_t id = a.gen_ids[i];
                if ((int64_t)id < V) atomicOr(&sh.u.bitmap[id >> 5], 1u << (id & 31));
            }
            __syncthreads();
        }
    }
    const double penf = (double)a.penalty;
    auto pval = [&](int64_t j, float xr) -> double {
        double v = (double)xr;
        if constexpr (!SIMPLE) {
            if (pen && ((sh.u.bitmap[j >> 5] >> (j & 31)) & 1u)) v = (v > 0.0) ? v / penf : v * penf;
        }
        return v;
    };
    auto val = [&](int64_t j) -> double { return pval(j, x[j]); };

    // ---- pass 1: max, first / last index of the max, NaN / +inf ---------
    double vmax = -INFINITY;
    int64_t ifirst = INT64_MAX, ilast = -1;
    uint32_t flg = 0;  // bit0 NaN, bit1 +inf
    NIS_G_EACH({
        const double v = pval(j, xr);
        const bool nan = v != v;
        flg |= nan ? 1u : 0u;
        flg |= (v == INFINITY) ? 2u : 0u;
        const bool gt = !nan && (ifirst == INT64_MAX || v > vmax);
        const bool eq = !nan && !gt && v == vmax;
        vmax = gt ? v : vmax;
        ifirst = gt ? j : ifirst;
        ilast = (gt || eq) ? j : ilast;
    })
    const double M = block_max(vmax, sh.dscr);
    ifirst = block_min(vmax == M ? ifirst : INT64_MAX, sh.iscr);
    ilast = block_max(vmax == M ? ilast : (int64_t)-1, sh.iscr);
    const uint64_t flags = block_or((uint64_t)flg, sh.uscr);
    const bool any_nan = flags & 1, any_pinf = flags & 2;
    const bool nan0 = (val(0) != val(0));

    // ---- greedy (sampler.rs:172-181): first index of the max; NaN skipped
    // by the strict `>` unless work[0] itself is NaN ----------------------
    if (a.temperature <= 0.0f) {
        if (tid == 0) {
            const uint32_t tok = (nan0 || ifirst == INT64_MAX) ? 0u : (uint32_t)ifirst;
            write_row_result(a, row, tok, NIS_PATH_GREEDY, 0.0, 0.0, 0.0, -1.0, 0.0, 0, 2, reject);
        }
        return true;
    }

    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const double M_w = M / temp;
    const float p = a.top_p;
    const bool topp_zero = (p <= 0.0f);
    const bool topp_on = (p > 0.0f) && (p < 1.0f);  // NaN p: neither branch

    // ---- a NaN row at top-p <= 0 without top-k (sampler.rs:122-134) -----
    // max_by hands the running maximum on at every comparison that is not
    // Greater, NaN on either side included, so the entry it keeps is the
    // last index of the maximum of w past the last NaN (at L), or L itself
    // when the NaN is the last entry.  Every other entry becomes -inf: a
    // finite kept value is drawn with mass 1 (index 0 when u = 0, as the
    // walk stops there), +inf is the non-finite-max argmax, and a kept NaN
    // or -inf returns 0.  (With top-k active the k-th value comes from a
    // sort whose comparator NaN makes inconsistent: not handled here.)
    if (any_nan && p <= 0.0f && !(a.top_k > 0 && a.top_k < (uint64_t)V)) {
        int64_t lnan = -1;
        NIS_G_EACH({ lnan = (pval(j, xr) != pval(j, xr)) ? max(lnan, j) : lnan; })
        lnan = block_max(lnan, sh.iscr);
        double smax = -INFINITY;
        int64_t slast = -1;
        NIS_G_EACH({
            if (j > lnan) {
                const double wv = pval(j, xr) / temp;  // sampler.rs:184-186
                const bool take = slast < 0 || wv > smax || (wv == smax && j > slast);
                smax = take ? wv : smax;
                slast = take ? j : slast;
            }
        })
        const double S = block_max(slast >= 0 ? smax : -INFINITY, sh.dscr);
        slast = block_max((slast >= 0 && smax == S) ? slast : (int64_t)-1, sh.iscr);
        const bool kept_nan = lnan == V - 1;
        const int64_t best = kept_nan ? lnan : slast;
        const double keep = kept_nan ? (double)NAN : S;
        if (w == 0) {
            if (keep > -INFINITY && keep < INFINITY) {
                uint64_t st[4];  // sampler.rs:209
                const uint64_t* sp = a.rng + 4 * (int64_t)row;
                st[0] = sp[0];
                st[1] = sp[1];
                st[2] = sp[2];
                st[3] = sp[3];
                const double u = rng_next_f64(st);
                if (l == 0) {
                    uint64_t* so = a.rng + 4 * (int64_t)row;
                    so[0] = st[0];
                    so[1] = st[1];
                    so[2] = st[2];
                    so[3] = st[3];
                    const uint32_t tok = (u == 0.0) ? 0u : (uint32_t)best;
                    write_row_result(a, row, tok, NIS_PATH_DRAW, keep, 1.0, 0.0, u,
                                     (tok == (uint32_t)best) ? 1.0 : 0.0, 1, 2, reject);
                }
            } else if (l == 0) {
                const uint32_t tok = (keep == INFINITY) ? (uint32_t)best : 0u;
                write_row_result(a, row, tok, NIS_PATH_NONFINITE_MAX, keep == INFINITY ? keep : -INFINITY, 0.0, 0.0, -1.0, 0.0,
                                 0, 2, reject);
            }
        }
        return true;
    }

    // ---- non-finite rows ------------------------------------------------
    // NaN survives every filter (all comparisons with NaN are false), so
    // `total` is NaN (sampler.rs:206) unless +inf makes the max non-finite
    // (sampler.rs:192), in which case the first-index argmax returns index 0
    // when work[0] is NaN and otherwise the first +inf.  With +inf and no
    // NaN, top-p removes nothing (its probabilities are NaN) except for
    // p <= 0, which keeps only the last maximum.  All -inf returns 0.
    if (any_nan || M == INFINITY || M == -INFINITY) {
        if (tid == 0) {
            uint32_t tok;
            uint32_t path;
            if (any_nan) {
                tok = (any_pinf && !nan0) ? (uint32_t)ifirst : 0u;
                path = (any_pinf || M == -INFINITY) ? NIS_PATH_NONFINITE_MAX : NIS_PATH_BAD_TOTAL;
            } else if (M == INFINITY) {
                tok = (uint32_t)(topp_zero ? ilast : ifirst);
                path = NIS_PATH_NONFINITE_MAX;
            } else {
                tok = 0u;
                path = NIS_PATH_NONFINITE_MAX;
            }
            write_row_result(a, row, tok, path, M_w, 0.0, 0.0, -1.0, 0.0, 0, 2, reject);
        }
        return true;
    }

    // Keys: penalised rows use the f64 key of w = v / T; other rows the f32
    // key of the logit (dividing by T > 0 preserves order and ties).
    auto keyof = [&](double v) -> uint64_t {
        if constexpr (SIMPLE) return (uint64_t)key32((float)v) << 32;
        else return pen ? key64(v / temp) : ((uint64_t)key32((float)v) << 32);
    };
    const uint64_t kmax = keyof(M);

    // Masses (see the header): 2^(x*c - R) octave by octave when the row has
    // no penalty and a finite reference; otherwise relative to the max,
    // 2^((w - M_w) log2 e).  `rho` turns the first form into units of the
    // max element.
    const double c64 = 1.4426950408889634 / temp;
    // c_hi rounded toward zero, so c_lo >= 0
    float cf = (float)c64;
    if ((double)cf > c64) cf = __uint_as_float(__float_as_uint(cf) - 1u);
    const float clo = (float)(c64 - (double)cf);
    const bool mf32 = !pen && fabsf((float)M * cf) < 1e30f;
    if (SIMPLE && !mf32) return false;  // nothing written yet
    const float Rf = mf32 ? ceilf((float)M * cf) : 0.0f;
    const int Ri = (int)Rf;
    // the position of x on the value grid: x*c - R in f32, monotone in x
    // (the histogram bins; within 2^-24 of its magnitude of the exponent)
    // (c_lo == 0 would turn x = -inf into NaN: then c_hi alone is c)
    auto tpos = [&](float xr) -> float {
        const float u = fmaf(xr, cf, -Rf);
        return clo != 0.0f ? fmaf(xr, clo, u) : u;
    };
    // 2^(x*c - R) as its octave mantissa fm = 2^(x*c - o) 2^24 rounded down
    // (f32 exp2 of the octave-relative argument, in [2^24, 2^25]) and e =
    // o - R: the mass is fm 2^(e - 24) exactly in f64, its 2^-40 fixed
    // point fm 2^(e + 16) (a shift).  fm = 0 for x = -inf; x is never NaN or
    // +inf here.
    auto mparts = [&](float xr, uint32_t& fm, int& e) {
        const float of = fminf(fmaxf(floorf(xr * cf), Rf - 1100.0f), Rf + 2.0f);
        const float f = fmaf(xr, clo, fmaf(xr, cf, -of));
        fm = xr > -INFINITY ? (uint32_t)(__builtin_amdgcn_exp2f(f) * 16777216.0f) : 0u;
        e = (int)of - Ri;
    };
    auto mfix = [](uint32_t fm, int e) -> unsigned long long {
        const int sh = e + 16;  // <= 18 (o <= R + 2)
        return sh >= 0 ? ((unsigned long long)fm << sh) : (sh > -32 ? (unsigned long long)(fm >> -sh) : 0ull);
    };
    auto massx = [&](float xr) -> double {
        uint32_t fm;
        int e;
        mparts(xr, fm, e);
        return ldexp((double)fm, e - 24);
    };
    auto fixx = [&](float xr) -> unsigned long long {  // floor(massx(x) 2^40)
        uint32_t fm;
        int e;
        mparts(xr, fm, e);
        return mfix(fm, e);
    };
    const double rho = mf32 ? 1.0 / massx((float)M) : 1.0;
    auto mass_w = [&](double wv) -> double {  // wv = value / T (penalised rows)
        const double t = (wv - M_w) * 1.4426950408889634;
        // far below f32's exp2 range (wv = -inf included, where t - th would
        // be NaN): mass 0
        if (!(t > -256.0)) return 0.0;
        const float th = (float)t;
        return (double)__builtin_amdgcn_exp2f(th) * (1.0 + (t - (double)th) * 0.6931471805599453);
    };
    auto massv = [&](double v, float xr) -> double {
        if constexpr (SIMPLE) return massx(xr);
        else return mf32 ? massx(xr) : mass_w(v / temp);
    };
    auto mass_of_key = [&](uint64_t k) -> double {
        const float xk = unkey32((uint32_t)(k >> 32));
        if constexpr (SIMPLE) return massx(xk);
        else {
            if (pen) return mass_w(unkey64(k));
            return mf32 ? massx(xk) : mass_w((double)xk / temp);
        }
    };

    // Bounds that skip an element before its key is computed (an f64
    // division on penalised rows) where it cannot matter: a lower bound on
    // the value of every element whose key is >= k (unpenalised rows key the
    // f32 logit, penalised ones the f64 value v / T), and an upper bound on
    // the value the penalty can give the logit x.
    auto vlb_of_key = [&](uint64_t k) -> double {
        if (!SIMPLE && pen) {
            const double wv = unkey64(k);  // every key >= k has v / T >= wv
            if (!(wv > -INFINITY) || !(wv < INFINITY)) return -INFINITY;
            const double b = wv * temp;
            return b - fabs(b) * 1.0e-12 - 1.0e-300;  // (v / T rounds: a margin)
        }
        const float f = unkey32((uint32_t)(k >> 32));
        return f == f ? (double)f : -INFINITY;
    };
    auto vub_of_x = [&](float xr) -> double {
        const double x = (double)xr;
        if (SIMPLE || !pen) return x;
        return x > 0.0 ? x * fmax(1.0, 1.0 / penf) * (1.0 + 1.0e-12)
                       : x * fmin(1.0, penf) * (1.0 - 1.0e-12);
    };

    // ---- top-k (sampler.rs:103-116): keep keys >= key of the k-th largest
    uint64_t kth = 0;
    const bool topk_on = a.top_k > 0 && a.top_k < (uint64_t)V;
    if (topk_on) {
        // On a penalised row the radix runs on keys of v itself (no division
        // per element) and its result converts once: w = v / T rounds
        // monotonically, so the k-th largest w is fl(v_k / T) for the k-th
        // largest v, ties the division creates included (they compare equal
        // as w-keys downstream).
        auto tkey = [&](double v) -> uint64_t {
            if constexpr (SIMPLE) return keyof(v);
            else return pen ? key64(v) : keyof(v);
        };
        auto vlb_of_tkey = [&](uint64_t k) -> double {
            if constexpr (!SIMPLE) {
                if (pen) {
                    const double v = unkey64(k);  // every key >= k has value >= v
                    return (v > -INFINITY && v < INFINITY) ? v : -INFINITY;
                }
            }
            return vlb_of_key(k);
        };
        const uint64_t tkmax = tkey(M);
        uint64_t diff = 0;
        NIS_G_EACH({ diff |= tkey(pval(j, xr)) ^ tkmax; })
        const DigitRange dr = digit_range(block_or(diff, sh.uscr));
        uint64_t prefix = (dr.hi_shift + 8 >= 64) ? 0 : (tkmax >> (dr.hi_shift + 8));
        uint64_t remaining = a.top_k;
        if (!dr.all_equal) {
            for (int shift = dr.hi_shift; shift >= dr.lo_shift; shift -= 8) {
                __syncthreads();
                if (tid < 256) sh.hcnt[tid] = 0;
                __syncthreads();
                // (an element whose value lies below every key of the prefix
                // cannot be in it)
                const double vlp = (shift + 8 >= 64) ? -INFINITY : vlb_of_tkey(prefix << (shift + 8));
                NIS_G_EACH({
                    if (vub_of_x(xr) >= vlp) {
                        const uint64_t k = tkey(pval(j, xr));
                        if (in_prefix(k, shift, prefix)) atomicAdd(&sh.hcnt[(k >> shift) & 255], 1u);
                    }
                })
                __syncthreads();
                if (w == 0) {
                    // the bucket holding the remaining-th largest key: the
                    // largest d whose count from the top reaches `remaining`
                    uint32_t cnt[4];
                    uint32_t lt = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        cnt[i] = sh.hcnt[4 * l + i];
                        lt += cnt[i];
                    }
                    const uint32_t incl = wscan_u32(lt);
                    const uint32_t tot = bcast_u32(incl, 63);
                    uint64_t fromtop = tot - incl;  // keys in higher lanes
                    int selb = -1;
                    uint64_t cum = 0;
#pragma unroll
                    for (int i = 3; i >= 0; --i) {
                        const bool hit = (fromtop + cnt[i] >= remaining) && selb < 0;
                        selb = hit ? (4 * l + i) : selb;
                        cum = hit ? fromtop : cum;
                        fromtop += cnt[i];
                    }
                    const int best = (int)wmax_f32((float)selb);  // highest d (exact in float)
                    const uint64_t own = __ballot(selb == best && best >= 0);
                    const int owner = own ? (__ffsll((long long)own) - 1) : 0;
                    const uint32_t cumb = bcast_u32((uint32_t)cum, owner);
                    if (l == 0) {
                        sh.bi[0] = best < 0 ? 0 : best;
                        sh.bi[1] = (int64_t)(remaining - cumb);
                    }
                }
                __syncthreads();
                prefix = (prefix << 8) | (uint64_t)sh.bi[0];
                remaining = (uint64_t)sh.bi[1];
            }
            const uint64_t lowmask = (dr.lo_shift == 0) ? 0 : ((1ull << dr.lo_shift) - 1);
            kth = (prefix << dr.lo_shift) | (tkmax & lowmask);
        } else {
            kth = tkmax;
        }
        if constexpr (!SIMPLE) {
            if (pen) kth = keyof(unkey64(kth));  // the k-th largest w = fl(v_k / T)
        }
    }

    // every element of value below vlb_kth has a key below the k-th's
    const double vlb_kth = topk_on ? vlb_of_key(kth) : -INFINITY;

    // ---- walk chunks: chunk c = elements [c*kGChunk, (c+1)*kGChunk), wave
    // c % kWaves; row e of it is elements c*kGChunk + 64e + (0..63), one per
    // lane (coalesced loads; index order is row by row, lane by lane) ----
    const int64_t nch = (V + kGChunk - 1) / kGChunk;
    auto load8 = [&](int64_t c, float* xs) {
        const int64_t j0 = c * kGChunk + l;
#pragma unroll
        for (int e = 0; e < 8; ++e) xs[e] = x[min(j0 + 64 * e, V - 1)];
    };
    bool sums_done = false;   // kept mass of every chunk already in csum[]
    int64_t kept_pre = 0;     // and the kept count of this thread

    // ---- top-p (sampler.rs:118-160) --------------------------------------
    double z_all = 0.0;
    uint64_t kstar = 0;      // keys > kstar kept; == kstar kept for tie rank < n_keep
    int64_t n_tie = 0, n_keep = 0;
    bool topp_done = false;
    if constexpr (SIMPLE) {
        if (topp_on && !topk_on) {
            // value histogram (count, fixed-point mass) with Z in one pass
#pragma unroll
            for (int i = 0; i < kGVBins / kBlock; ++i) {
                sh.u.v.cnt[tid + i * kBlock] = 0u;
                sh.u.v.mass[tid + i * kBlock] = 0ull;
            }
            __syncthreads();
            auto vbin = [&](float t) -> uint32_t {
                return (uint32_t)fminf(fmaxf(-t * kGVRes, 0.0f), (float)(kGVBins - 1));
            };
            double zl = 0.0;
            NIS_G_EACH({
                (void)j;  // (the bin needs the value only)
                const float t = tpos(xr);
                uint32_t fm;
                int me;
                mparts(xr, fm, me);
                zl += ldexp((double)fm, me - 24);
                const uint32_t b = vbin(t);
                atomicAdd(&sh.u.v.cnt[b], 1u);
                atomicAdd(&sh.u.v.mass[b], mfix(fm, me));
            })
            z_all = block_sum(zl, sh.dscr);
            const double pZ = (double)p * z_all;
            // wave 0: the lowest bin b_a passing sampler.rs:150 with the bin's
            // upper edge 2^(-b/kGVRes) for its first element, raised by 2^-17
            // for the bin position's rounding (at most 2^-24 of 64 octaves).
            // That edge is at least the first element's mass, so the true
            // cutoff bin is b_a or the nonempty bin b_p above it; their
            // members are listed next.
            if (w == 0) {
                constexpr int per = kGVBins / 64;
                unsigned long long ltot = 0;
#pragma unroll 8
                for (int i = 0; i < per; ++i) ltot += sh.u.v.mass[per * l + i];
                const double incl = wscan_f64((double)ltot);
                double above = incl - (double)ltot;  // fixed point, bins of lower lanes
                int ba = -1;
#pragma unroll 8
                for (int i = 0; i < per; ++i) {
                    const int b = per * l + i;
                    const uint32_t n = sh.u.v.cnt[b];
                    const double G = above / kGFix;
                    const double edge =
                        (double)__builtin_amdgcn_exp2f(-(float)b / kGVRes) * (1.0 + 0x1p-17);
                    const bool q = (n != 0) && (G - edge <= pZ);
                    ba = q ? b : ba;
                    above += (double)sh.u.v.mass[b];
                }
                const int bA = (int)wmax_f32((float)ba);  // highest qualifying bin (exact in float)
                // b_p: the last nonempty bin above b_A, and the mass above it
                int lp = -1;
                double gp = 0.0;
                above = incl - (double)ltot;
#pragma unroll 8
                for (int i = 0; i < per; ++i) {
                    const int b = per * l + i;
                    const bool ne = sh.u.v.cnt[b] != 0;
                    const bool take = ne && b < bA;
                    lp = take ? b : lp;
                    gp = take ? above / kGFix : gp;
                    above += (double)sh.u.v.mass[b];
                }
                const int bP = (int)wmax_f32((float)lp);
                const uint64_t own = __ballot(lp == bP && bP >= 0);
                const int owner = own ? (__ffsll((long long)own) - 1) : 0;
                const double G0 = (bP >= 0) ? bcast_f64(gp, owner) : 0.0;
                if (l == 0) {
                    sh.bi[0] = bA;
                    sh.bi[1] = bP;
                    sh.bd[0] = G0;
                }
            }
            __syncthreads();
            const int bA = (int)sh.bi[0], bP = (int)sh.bi[1];
            const double G0 = sh.bd[0];
            if (bA >= 0) {
                // one pass over the walk chunks: the mass of the elements
                // above bin b_p (all kept) per chunk, and lane-private lists
                // of the members of bins b_p and b_a
                int nlane = 0;
                int64_t nsure = 0;
                uint64_t diff = 0;
                const uint32_t kref = (uint32_t)(kmax >> 32);
                const int bTop = (bP >= 0) ? bP : bA;  // bins above it hold kept elements only
                float xn8[8];
                if (w < nch) load8(w, xn8);
                for (int64_t cc = w; cc < nch; cc += kWaves) {
                    float xs[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) xs[e] = xn8[e];
                    load8(min(cc + kWaves, nch - 1), xn8);  // the next chunk, in flight meanwhile
                    double sl = 0.0;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int64_t j = cc * kGChunk + 64 * e + l;
                        const bool inr = j < V;
                        const float t = tpos(xs[e]);
                        const int b = (int)vbin(t);
                        const bool sure = inr & (b < bTop);
                        sl += sure ? massx(xs[e]) : 0.0;
                        nsure += sure ? 1 : 0;
                        const bool in = inr & ((b == bA) | (b == bP));
                        diff |= in ? ((uint64_t)(key32(xs[e]) ^ kref) << 32) : 0ull;
                        if (in) {
                            if (nlane < kGLane) {
                                sh.u.v.lx[nlane][tid] = xs[e];
                                sh.u.v.li[nlane][tid] = (uint32_t)j;
                            }
                            ++nlane;
                        }
                    }
                    const double cs = wsum_f64(sl);
                    if (l == 0) sh.csum[cc] = (unsigned long long)(cs * kGFix);
                }
                const int64_t novf = block_sum((int64_t)(nlane > kGLane ? 1 : 0), sh.iscr);
                if (novf == 0) {
                    // the radix walk of the general form, over the listed members
                    const DigitRange dr = digit_range(block_or(diff, sh.uscr));
                    uint64_t prefix = (dr.hi_shift + 8 >= 64) ? 0 : (kmax >> (dr.hi_shift + 8));
                    double G = G0;
                    if (!dr.all_equal) {
                        for (int shift = dr.hi_shift; shift >= dr.lo_shift; shift -= 8) {
                            __syncthreads();
                            if (tid < 256) {
                                sh.hcnt[tid] = 0;
                                sh.hmass[tid] = 0ull;
                                sh.hkey[tid] = 0ull;
                            }
                            __syncthreads();
                            for (int i = 0; i < nlane; ++i) {
                                const float xl = sh.u.v.lx[i][tid];
                                const uint64_t k = (uint64_t)key32(xl) << 32;
                                if (in_prefix(k, shift, prefix)) {
                                    const int d = (int)((k >> shift) & 255);
                                    atomicAdd(&sh.hcnt[d], 1u);
                                    atomicAdd(&sh.hmass[d], fixx(xl));
                                    atomicMax(&sh.hkey[d], (unsigned long long)k);
                                }
                            }
                            __syncthreads();
                            if (w == 0) {
                                int sel;
                                double gsel;
                                uint32_t nsel;
                                topp_digit_select(sh, G, pZ, mass_of_key, &sel, &gsel, &nsel);
                                if (l == 0) {
                                    sh.bi[0] = sel < 256 ? sel : 0;
                                    sh.bi[1] = sel < 256 ? (int64_t)nsel : 0;
                                    sh.bd[0] = sel < 256 ? gsel : G;
                                }
                            }
                            __syncthreads();
                            prefix = (prefix << 8) | (uint64_t)sh.bi[0];
                            G = sh.bd[0];
                            n_tie = sh.bi[1];
                        }
                        const uint64_t lowmask = (dr.lo_shift == 0) ? 0 : ((1ull << dr.lo_shift) - 1);
                        kstar = (prefix << dr.lo_shift) | (kmax & lowmask);
                    } else {
                        // every listed member has the key of the row max
                        kstar = kmax;
                        n_tie = block_sum((int64_t)nlane, sh.iscr);
                    }
                    const double es = mass_of_key(kstar);
                    const double q = (pZ - G) / es;  // >= -1 for the selected key
                    if (!(q < (double)n_tie)) n_keep = n_tie;
                    else n_keep = min(n_tie, (int64_t)floor(q) + 2);
                    if (n_keep < 1) n_keep = 1;
                    topp_done = true;
                    if (n_keep >= n_tie) {
                        // no tie group split: the kept listed members join the
                        // mass of their chunks (fixed point, exact)
                        int64_t nkl = 0;
                        for (int i = 0; i < nlane; ++i) {
                            const float xl = sh.u.v.lx[i][tid];
                            const uint64_t k = (uint64_t)key32(xl) << 32;
                            if (k >= kstar) {
                                const uint32_t jl = sh.u.v.li[i][tid];
                                atomicAdd(&sh.csum[jl / kGChunk], fixx(xl));
                                ++nkl;
                            }
                        }
                        kept_pre = nsure + nkl;
                        sums_done = true;
                    }
                }
            }
            __syncthreads();
        }
    }
    double vlb_p = -INFINITY;  // (top-p on the general form) no element below it is kept
    if (topp_on && !topp_done) {
        double zl = 0.0;
        uint64_t diff = 0;
        NIS_G_EACH({
            if (vub_of_x(xr) >= vlb_kth) {
                const double v = pval(j, xr);
                const uint64_t k = keyof(v);
                const bool live = k >= kth;
                zl += live ? massv(v, xr) : 0.0;
                diff |= live ? (k ^ kmax) : 0ull;
            }
        })
        z_all = block_sum(zl, sh.dscr);
        const DigitRange dr = digit_range(block_or(diff, sh.uscr));
        const double pZ = (double)p * z_all;
        // sampler.rs:150 removes an element of mass m, whatever the others,
        // once (V + 1) m < (1 - p) Z: the mass at or below it and its own are
        // then less than (1 - p) Z, so the mass before it exceeds p Z plus its
        // own.  Every element whose value lies below vlb_p (a 16-fold margin
        // on that mass) is removed, and the passes below skip it before its
        // key is computed (on a penalised row of N(0, 3) logits at T 0.8 and
        // p 0.9, ~90 % of the row).
        {
            const double mrel = (1.0 - (double)p) * z_all * rho / (16.0 * (double)V);
            if (mrel > 0.0 && mrel < 1.0 && M_w > -INFINITY && M_w < INFINITY) {
                const double b = temp * (M_w + log(mrel));
                vlb_p = b - fabs(b) * 1.0e-12 - 1.0e-300;
            }
        }
        const double vlb = fmax(vlb_kth, vlb_p);
        uint64_t prefix = (dr.hi_shift + 8 >= 64) ? 0 : (kmax >> (dr.hi_shift + 8));
        double G = 0.0;
        if (!dr.all_equal) {
            for (int shift = dr.hi_shift; shift >= dr.lo_shift; shift -= 8) {
                __syncthreads();
                if (tid < 256) {
                    sh.hcnt[tid] = 0;
                    sh.hmass[tid] = 0ull;
                    sh.hkey[tid] = 0ull;
                }
                __syncthreads();
                NIS_G_EACH({
                    if (vub_of_x(xr) >= vlb) {  // (below the k-th: not live; below vlb_p: removed)
                        const double v = pval(j, xr);
                        const uint64_t k = keyof(v);
                        if (k >= kth && in_prefix(k, shift, prefix)) {
                            const int d = (int)((k >> shift) & 255);
                            atomicAdd(&sh.hcnt[d], 1u);
                            atomicAdd(&sh.hmass[d], (unsigned long long)(massv(v, xr) * kGFix));
                            atomicMax(&sh.hkey[d], (unsigned long long)k);
                        }
                    }
                })
                __syncthreads();
                if (w == 0) {
                    int sel;
                    double gsel;
                    uint32_t nsel;
                    topp_digit_select(sh, G, pZ, mass_of_key, &sel, &gsel, &nsel);
                    if (l == 0) {
                        // sel < 256: a bucket holds a kept element (the first
                        // key of the current range always is)
                        sh.bi[0] = sel < 256 ? sel : 0;
                        sh.bi[1] = sel < 256 ? (int64_t)nsel : 0;
                        sh.bd[0] = sel < 256 ? gsel : G;
                    }
                }
                __syncthreads();
                prefix = (prefix << 8) | (uint64_t)sh.bi[0];
                G = sh.bd[0];
                n_tie = sh.bi[1];
            }
            const uint64_t lowmask = (dr.lo_shift == 0) ? 0 : ((1ull << dr.lo_shift) - 1);
            kstar = (prefix << dr.lo_shift) | (kmax & lowmask);
        } else {
            kstar = kmax;
            int64_t cnt = 0;
            NIS_G_EACH({ cnt += (keyof(pval(j, xr)) == kmax) ? 1 : 0; })
            n_tie = block_sum(cnt, sh.iscr);
        }
        const double es = mass_of_key(kstar);
        const double q = (pZ - G) / es;  // >= -1 for the selected key
        if (!(q < (double)n_tie)) n_keep = n_tie;
        else n_keep = min(n_tie, (int64_t)floor(q) + 2);
        if (n_keep < 1) n_keep = 1;
    }

    // kept(j): the final filtered set of sampler.rs:187-188
    // mode 0: live (top-k survivors); 1: top-p prefix; 2: p <= 0, last max
    const int mode = topp_zero ? 2 : (topp_on ? 1 : 0);
    const bool tie_split = (mode == 1) && (n_keep < n_tie);

    // tie-group members (key == kstar) before each chunk, when only some of
    // them are kept (ties are kept in ascending index order)
    if (tie_split) {
        for (int64_t cc = w; cc < nch; cc += kWaves) {
            float xs[8];
            load8(cc, xs);
            uint32_t tl = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t j = cc * kGChunk + 64 * e + l;
                tl += (j < V && vub_of_x(xs[e]) >= vlb_p && keyof(pval(j, xs[e])) == kstar) ? 1u : 0u;
            }
            const uint32_t tc = wsum_u32(tl);
            if (l == 0) sh.tcnt[cc] = tc;
        }
        __syncthreads();
        if (w == 0) {  // exclusive prefix over the chunks, in place
            uint32_t run = 0;
            for (int64_t c0 = 0; c0 < nch; c0 += 64) {
                const int64_t cc = c0 + l;
                const uint32_t v = (cc < nch) ? sh.tcnt[cc] : 0u;
                const uint32_t inc = wscan_u32(v);
                if (cc < nch) sh.tcnt[cc] = run + inc - v;
                run += bcast_u32(inc, 63);
            }
        }
        __syncthreads();
    }
    // kept flags and masses of a lane's 8 elements (one per row) of chunk cc
    auto chunk_kept = [&](int64_t cc, const float* xs, uint32_t tie_base, double* e8,
                          uint32_t* kmask) {
        uint32_t rowbase = tie_base;  // tie members before this row
        uint32_t km = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t j = cc * kGChunk + 64 * e + l;
            const bool in = j < V;
            // (an element below the k-th's value gets key 0: below kth, not kept)
            double v = -INFINITY;
            uint64_t k = 0ull;
            if (vub_of_x(xs[e]) >= vlb_kth && (mode != 1 || vub_of_x(xs[e]) >= vlb_p)) {
                v = pval(j, xs[e]);
                k = keyof(v);
            }
            bool kp;
            if (mode == 2) kp = (j == ilast);
            else if (k < kth) kp = false;
            else if (mode == 0) kp = true;
            else if (k > kstar) kp = true;
            else if (k < kstar) kp = false;
            else kp = true;
            if (tie_split) {  // ties are kept in ascending index order
                const bool tie = in && k == kstar;
                const uint64_t mt = __ballot(tie);
                const uint32_t tr = rowbase + lane_rank(mt);
                kp = tie ? ((int64_t)tr < n_keep) : kp;
                rowbase += (uint32_t)__popcll(mt);
            }
            // (a -inf survivor of top-k or of top-p off has mass 0: it can
            // never end the walk, and the kept count, like the reference's
            // finite survivors, leaves it out)
            kp = kp && in && (v > -INFINITY);
            km |= kp ? (1u << e) : 0u;
            e8[e] = kp ? massv(v, xs[e]) : 0.0;
        }
        *kmask = km;
    };

    // ---- kept mass of every chunk ----------------------------------------
    int64_t nk = kept_pre;
    float xn8[8];
    if (!sums_done && w < nch) load8(w, xn8);
    for (int64_t cc = w; cc < nch && !sums_done; cc += kWaves) {
        float xs[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) xs[e] = xn8[e];
        load8(min(cc + kWaves, nch - 1), xn8);  // the next chunk, in flight meanwhile
        double e8[8];
        uint32_t km;
        chunk_kept(cc, xs, tie_split ? sh.tcnt[cc] : 0u, e8, &km);
        double s = 0.0;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += e8[e];
        nk += __popc(km);
        const double cs = wsum_f64(s);
        if (l == 0) sh.csum[cc] = (unsigned long long)(cs * kGFix);
    }
    const int64_t kept_total = block_sum(nk, sh.iscr);  // contains a barrier: csum[] visible after it

    // ---- wave 0: the total, the draw, the chunk, lane and element of the
    // crossing (sampler.rs:209-216) -----------------------------------------
    if (w != 0) return true;
    const int64_t per = (nch + 63) / 64;  // chunks per lane, in order
    double ls = 0.0;
    for (int64_t i = 0; i < per; ++i) {
        const int64_t cc = (int64_t)l * per + i;
        ls += (cc < nch) ? (double)sh.csum[cc] / kGFix : 0.0;
    }
    const double lincl = wscan_f64(ls);
    const double z_kept = bcast_f64(lincl, 63);
    const double zkM = z_kept * rho, zaM = z_all * rho;
    if (!(z_kept > 0.0) || !(z_kept < INFINITY)) {  // sampler.rs:206-208
        if (l == 0)
            write_row_result(a, row, 0u, NIS_PATH_BAD_TOTAL, M_w, zkM, zaM, -1.0, 0.0,
                             (uint64_t)kept_total, 2, reject);
        return true;
    }
    uint64_t st[4];  // sampler.rs:209 — the only RNG advance of the call
    {
        const uint64_t* sp = a.rng + 4 * (int64_t)row;
        st[0] = sp[0];
        st[1] = sp[1];
        st[2] = sp[2];
        st[3] = sp[3];
    }
    const double u = rng_next_f64(st);
    if (l == 0) {
        uint64_t* sp = a.rng + 4 * (int64_t)row;
        sp[0] = st[0];
        sp[1] = st[1];
        sp[2] = st[2];
        sp[3] = st[3];
    }
    const double r = u * z_kept;
    // the lane whose chunks hold the crossing: the first whose running total
    // reaches r with mass of its own; rounding: the last lane with mass
    const uint64_t hl = __ballot((lincl >= r) & (ls > 0.0));
    const uint64_t nzl = __ballot(ls > 0.0);
    const int L = hl ? (__ffsll((long long)hl) - 1) : (63 - __clzll((long long)nzl));
    int64_t csel = -1, clast = -1;
    double cbase = 0.0, clbase = 0.0;
    {
        double run = bcast_f64(lincl - ls, L);
        for (int64_t i = 0; i < per; ++i) {
            const int64_t cc = (int64_t)L * per + i;
            const double v = (cc < nch) ? (double)sh.csum[cc] / kGFix : 0.0;
            if (v > 0.0 && csel < 0) {
                clast = cc;
                clbase = run;
                if (run + v >= r) {
                    csel = cc;
                    cbase = run;
                }
            }
            run += v;
        }
    }
    if (csel < 0) {  // rounding: the last chunk with mass
        csel = clast;
        cbase = clbase;
    }
    // the chunk's 8 rows: the row holding the crossing (row totals), then
    // the lane inside it (prefix over the row's 64 elements)
    float xs[8];
    load8(csel, xs);
    double e8[8];
    uint32_t km;
    chunk_kept(csel, xs, tie_split ? sh.tcnt[csel] : 0u, e8, &km);
    int rsel = -1, rlast = -1;
    double rbase = cbase, rlbase = cbase;
    {
        double run = cbase;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const double rs = wsum_f64(e8[e]);
            const bool nzr = rs > 0.0;
            const bool first = nzr && rsel < 0;
            rlast = first ? e : rlast;
            rlbase = first ? run : rlbase;
            const bool hitr = first && (run + rs >= r);
            rsel = hitr ? e : rsel;
            rbase = hitr ? run : rbase;
            run += rs;
        }
    }
    if (rsel < 0) {  // rounding: the last row with mass
        rsel = rlast;
        rbase = rlbase;
    }
    double er = e8[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) er = (e == rsel) ? e8[e] : er;
    const double rincl = wscan_f64(er);
    const uint64_t hit = __ballot((rbase + rincl >= r) & (er > 0.0));
    const uint64_t nz = __ballot(er > 0.0);
    const bool rounded = hit == 0;  // rounding: the row's last kept element
    const int LL = hit ? (__ffsll((long long)hit) - 1) : (63 - __clzll((long long)nz));
    if (l == LL) {
        int64_t tok = csel * kGChunk + 64 * rsel + l;
        const double etok = er;
        bool ktok = true;
        (void)rounded;
        if (u == 0.0) {  // r == 0 stops the reference's walk at index 0
            tok = 0;
            ktok = false;
        }
        write_row_result(a, row, (uint32_t)tok, NIS_PATH_DRAW, M_w, zkM, zaM, u,
                         ktok ? etok / z_kept : 0.0, (uint64_t)kept_total, 2, reject);
    }
    return true;
}
#undef NIS_G_EACH

// The general path: the SIMPLE form (f32 masses, no penalty lookups in the
// passes) when it applies, else the general one.
template <int TAG = 0>
__device__ __forceinline__ void general_row(const RowArgs a, const int row, GeneralShared& sh,
                                            const uint32_t reject) {
    if (!general_row_t<true, TAG>(a, row, sh, reject)) {
        __syncthreads();
        general_row_t<false, TAG>(a, row, sh, reject);
    }
}

}  // namespace nis
