// general_path.h — the general per-row sampler: one 1024-lane workgroup per
// row, any V <= NIS_MAX_V, repetition penalty, top-k, top-p and every
// special case of sample() (src/sampler.rs:163-217).  It makes several
// passes over the row (re-read through L2 / MALL), computes in f64 with the
// device libm `exp`, and is used for rows the register-resident fast path
// does not take (penalty, top-k, non-finite input, V above its capacity).
//
// Sort-free top-p (sampler.rs:118-160): the reference keeps sorted position
// pos iff D(pos) = cum_excl(pos) - q(pos) <= p (normalised).  D is
// non-decreasing in pos, so the kept set is a prefix of the stable order.
// A most-significant-digit radix walk over order-preserving keys carries
// G = mass strictly above the current key range and picks, per digit, the
// last bucket whose first (largest-key) element is kept: G - e_first <= p*Z.
// At the last digit the bucket is one key value K*, i.e. a tie group whose
// members are kept in ascending index order while G + (j-1)*e* <= p*Z.
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
    const int64_t* gen_off;
    uint32_t* tokens;
    nis_row_stats* stats;
};

struct GeneralShared {
    uint32_t bitmap[NIS_MAX_V / 32];  // penalised-id set of the row
    uint32_t hcnt[256];
    double hmass[256];
    unsigned long long hkey[256];
    double incl[kBlock];              // per-thread inclusive kept-mass prefix
    double dscr[kWaves];
    uint64_t uscr[kWaves];
    int64_t iscr[kWaves];
    double bd[4];
    int64_t bi[4];
};

__device__ __forceinline__ void write_row_result(const RowArgs a, int row, uint32_t token,
                                                 uint32_t path, double max_w, double z_kept,
                                                 double z_all, double u, double prob,
                                                 uint64_t kept, uint32_t kernel,
                                                 uint32_t reject = NIS_REJECT_NONE) {
    a.tokens[row] = token;
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

// `reject` is recorded in the row's stats: why the fast path declined it.
__device__ __noinline__ void general_row(const RowArgs a, const int row, GeneralShared& sh,
                                         const uint32_t reject) {
    const int tid = threadIdx.x;
    const float* __restrict__ x = a.logits + (int64_t)row * a.ld;
    const int64_t V = a.V;

    // ---- repetition penalty set (sampler.rs:83-101) --------------------
    bool pen = false;
    if (a.penalty != 1.0f && a.gen_ids != nullptr && a.gen_off != nullptr) {
        const int64_t g0 = a.gen_off[row], g1 = a.gen_off[row + 1];
        if (g1 > g0) {
            pen = true;
            const int64_t nw = (V + 31) >> 5;
            for (int64_t i = tid; i < nw; i += kBlock) sh.bitmap[i] = 0u;
            __syncthreads();
            for (int64_t i = g0 + tid; i < g1; i += kBlock) {
                const uint32_t id = a.gen_ids[i];
                if ((int64_t)id < V) atomicOr(&sh.bitmap[id >> 5], 1u << (id & 31));
            }
            __syncthreads();
        }
    }
    const double penf = (double)a.penalty;
    auto val = [&](int64_t j) -> double {
        double v = (double)x[j];
        if (pen && ((sh.bitmap[j >> 5] >> (j & 31)) & 1u)) v = (v > 0.0) ? v / penf : v * penf;
        return v;
    };

    // ---- pass 1: max, first / last index of the max, NaN / +inf ---------
    double vmax = -INFINITY;
    int64_t ifirst = INT64_MAX, ilast = -1;
    uint64_t flags = 0;  // bit0 NaN, bit1 +inf
    for (int64_t j = tid; j < V; j += kBlock) {
        const double v = val(j);
        if (v != v) {
            flags |= 1;
            continue;
        }
        if (ifirst == INT64_MAX || v > vmax) {
            vmax = v;
            ifirst = j;
            ilast = j;
        } else if (v == vmax) {
            ilast = j;
        }
        if (v == INFINITY) flags |= 2;
    }
    const double M = block_max(vmax, sh.dscr);
    ifirst = block_min(vmax == M ? ifirst : INT64_MAX, sh.iscr);
    ilast = block_max(vmax == M ? ilast : (int64_t)-1, sh.iscr);
    flags = block_or(flags, sh.uscr);
    const bool any_nan = flags & 1, any_pinf = flags & 2;
    const bool nan0 = (val(0) != val(0));

    // ---- greedy (sampler.rs:172-181): first index of the max; NaN skipped
    // by the strict `>` unless work[0] itself is NaN ----------------------
    if (a.temperature <= 0.0f) {
        if (tid == 0) {
            const uint32_t tok = (nan0 || ifirst == INT64_MAX) ? 0u : (uint32_t)ifirst;
            write_row_result(a, row, tok, NIS_PATH_GREEDY, 0.0, 0.0, 0.0, -1.0, 0.0, 0, 2, reject);
        }
        return;
    }

    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const double M_w = M / temp;
    const float p = a.top_p;
    const bool topp_zero = (p <= 0.0f);
    const bool topp_on = (p > 0.0f) && (p < 1.0f);  // NaN p: neither branch

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
        return;
    }

    // Keys: penalised rows use the f64 key of w = v / T; other rows the f32
    // key of the logit (dividing by T > 0 preserves order and ties).
    auto keyof = [&](double v) -> uint64_t {
        return pen ? key64(v / temp) : ((uint64_t)key32((float)v) << 32);
    };
    auto key_w = [&](uint64_t k) -> double {
        return pen ? unkey64(k) : (double)unkey32((uint32_t)(k >> 32)) / temp;
    };
    const uint64_t kmax = keyof(M);

    // ---- top-k (sampler.rs:103-116): keep keys >= key of the k-th largest
    uint64_t kth = 0;
    const bool topk_on = a.top_k > 0 && a.top_k < (uint64_t)V;
    if (topk_on) {
        uint64_t diff = 0;
        for (int64_t j = tid; j < V; j += kBlock) diff |= keyof(val(j)) ^ kmax;
        const DigitRange dr = digit_range(block_or(diff, sh.uscr));
        uint64_t prefix = (dr.hi_shift + 8 >= 64) ? 0 : (kmax >> (dr.hi_shift + 8));
        uint64_t remaining = a.top_k;
        if (!dr.all_equal) {
            for (int shift = dr.hi_shift; shift >= dr.lo_shift; shift -= 8) {
                __syncthreads();
                if (tid < 256) sh.hcnt[tid] = 0;
                __syncthreads();
                for (int64_t j = tid; j < V; j += kBlock) {
                    const uint64_t k = keyof(val(j));
                    if (in_prefix(k, shift, prefix)) atomicAdd(&sh.hcnt[(k >> shift) & 255], 1u);
                }
                __syncthreads();
                if (tid == 0) {
                    uint64_t cum = 0;
                    int sel = 0;
                    for (int d = 255; d >= 0; --d) {
                        if (cum + sh.hcnt[d] >= remaining) {
                            sel = d;
                            break;
                        }
                        cum += sh.hcnt[d];
                    }
                    sh.bi[0] = sel;
                    sh.bi[1] = (int64_t)(remaining - cum);
                }
                __syncthreads();
                prefix = (prefix << 8) | (uint64_t)sh.bi[0];
                remaining = (uint64_t)sh.bi[1];
            }
            const uint64_t lowmask = (dr.lo_shift == 0) ? 0 : ((1ull << dr.lo_shift) - 1);
            kth = (prefix << dr.lo_shift) | (kmax & lowmask);
        } else {
            kth = kmax;
        }
    }

    // ---- top-p (sampler.rs:118-160) --------------------------------------
    double z_all = 0.0;
    uint64_t kstar = 0;      // keys > kstar kept; == kstar kept for tie rank < n_keep
    int64_t n_tie = 0, n_keep = 0;
    if (topp_on) {
        double zl = 0.0;
        uint64_t diff = 0;
        for (int64_t j = tid; j < V; j += kBlock) {
            const double v = val(j);
            const uint64_t k = keyof(v);
            if (k < kth) continue;
            zl += exp(v / temp - M_w);
            diff |= k ^ kmax;
        }
        z_all = block_sum(zl, sh.dscr);
        const DigitRange dr = digit_range(block_or(diff, sh.uscr));
        const double pZ = (double)p * z_all;
        uint64_t prefix = (dr.hi_shift + 8 >= 64) ? 0 : (kmax >> (dr.hi_shift + 8));
        double G = 0.0;
        if (!dr.all_equal) {
            for (int shift = dr.hi_shift; shift >= dr.lo_shift; shift -= 8) {
                __syncthreads();
                if (tid < 256) {
                    sh.hcnt[tid] = 0;
                    sh.hmass[tid] = 0.0;
                    sh.hkey[tid] = 0ull;
                }
                __syncthreads();
                for (int64_t j = tid; j < V; j += kBlock) {
                    const double v = val(j);
                    const uint64_t k = keyof(v);
                    if (k < kth || !in_prefix(k, shift, prefix)) continue;
                    const int d = (int)((k >> shift) & 255);
                    atomicAdd(&sh.hcnt[d], 1u);
                    atomicAdd(&sh.hmass[d], exp(v / temp - M_w));
                    atomicMax(&sh.hkey[d], (unsigned long long)k);
                }
                __syncthreads();
                if (tid == 0) {
                    double g = G, g_sel = G;
                    int sel = -1;
                    for (int d = 255; d >= 0; --d) {
                        if (sh.hcnt[d] == 0) continue;
                        const double ef = exp(key_w(sh.hkey[d]) - M_w);
                        if (g - ef <= pZ) {
                            sel = d;
                            g_sel = g;
                            g += sh.hmass[d];
                        } else {
                            break;
                        }
                    }
                    sh.bi[0] = sel < 0 ? 0 : sel;  // sel >= 0: the first bucket holds a kept element
                    sh.bi[1] = sel < 0 ? 0 : sh.hcnt[sel];
                    sh.bd[0] = g_sel;
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
            for (int64_t j = tid; j < V; j += kBlock) cnt += (keyof(val(j)) == kmax) ? 1 : 0;
            n_tie = block_sum(cnt, sh.iscr);
        }
        const double es = exp(key_w(kstar) - M_w);
        const double q = (pZ - G) / es;  // >= -1 for the selected key
        if (!(q < (double)n_tie)) n_keep = n_tie;
        else n_keep = min(n_tie, (int64_t)floor(q) + 2);
        if (n_keep < 1) n_keep = 1;
    }

    // kept(j): the final filtered set of sampler.rs:187-188
    // mode 0: live (top-k survivors); 1: top-p prefix; 2: p <= 0, last max
    const int mode = topp_zero ? 2 : (topp_on ? 1 : 0);
    const bool tie_split = (mode == 1) && (n_keep < n_tie);

    // ---- contiguous index ranges for the in-order walk ------------------
    const int64_t L = (V + kBlock - 1) / kBlock;
    const int64_t j0 = min((int64_t)tid * L, V), j1 = min(j0 + L, V);

    int64_t tie_base = 0;
    if (tie_split) {
        int64_t c = 0;
        for (int64_t j = j0; j < j1; ++j) c += (keyof(val(j)) == kstar) ? 1 : 0;
        int64_t tot;
        const int64_t inc = block_inclusive_scan(c, sh.iscr, &tot);
        tie_base = inc - c;
    }
    auto kept_at = [&](int64_t j, uint64_t k, int64_t& tie_rank) -> bool {
        if (mode == 2) return j == ilast;
        if (k < kth) return false;
        if (mode == 0) return true;
        if (k > kstar) return true;
        if (k < kstar) return false;
        const bool keep = tie_rank < n_keep;
        ++tie_rank;
        return keep;
    };

    double s = 0.0;
    int64_t nk = 0;
    {
        int64_t tr = tie_base;
        for (int64_t j = j0; j < j1; ++j) {
            const double v = val(j);
            const uint64_t k = keyof(v);
            if (kept_at(j, k, tr)) {
                s += exp(v / temp - M_w);
                ++nk;
            }
        }
    }
    double z_kept;
    const double I = block_inclusive_scan(s, sh.dscr, &z_kept);
    sh.incl[tid] = I;
    const int64_t kept_total = block_sum(nk, sh.iscr);  // contains a barrier: incl[] visible after it

    if (!(z_kept > 0.0) || !(z_kept < INFINITY)) {  // sampler.rs:206-208
        if (tid == 0)
            write_row_result(a, row, 0u, NIS_PATH_BAD_TOTAL, M_w, z_kept, z_all, -1.0, 0.0,
                             (uint64_t)kept_total, 2, reject);
        return;
    }
    if (tid == 0) {  // sampler.rs:209 — the only RNG advance of the call
        uint64_t st[4];
        uint64_t* sp = a.rng + 4 * (int64_t)row;
        st[0] = sp[0];
        st[1] = sp[1];
        st[2] = sp[2];
        st[3] = sp[3];
        sh.bd[1] = rng_next_f64(st);
        sp[0] = st[0];
        sp[1] = st[1];
        sp[2] = st[2];
        sp[3] = st[3];
    }
    __syncthreads();
    const double u = sh.bd[1];
    const double r = u * z_kept;
    // first thread whose inclusive prefix reaches r (exists: r < z_kept)
    const int64_t tsel = block_min((I >= r) ? (int64_t)tid : (int64_t)INT64_MAX, sh.iscr);
    if ((int64_t)tid == tsel) {
        double run = (tid == 0) ? 0.0 : sh.incl[tid - 1];
        int64_t tr = tie_base;
        int64_t tok = -1, last_kept = -1;
        double etok = 0.0;
        bool ktok = false;
        for (int64_t j = j0; j < j1; ++j) {
            const double v = val(j);
            const uint64_t k = keyof(v);
            const bool kp = kept_at(j, k, tr);
            double e = 0.0;
            if (kp) {
                e = exp(v / temp - M_w);
                run += e;
                last_kept = j;
            }
            if (run >= r) {  // sampler.rs:211-213: r -= w; if r <= 0 return i
                tok = j;
                etok = e;
                ktok = kp;
                break;
            }
        }
        if (tok < 0) {  // rounding: the crossing is the range's last kept token
            tok = last_kept;
            ktok = true;
            etok = exp(val(tok) / temp - M_w);
        }
        write_row_result(a, row, (uint32_t)tok, NIS_PATH_DRAW, M_w, z_kept, z_all, u,
                         ktok ? etok / z_kept : 0.0, (uint64_t)kept_total, 2, reject);
    }
}

}  // namespace nis
