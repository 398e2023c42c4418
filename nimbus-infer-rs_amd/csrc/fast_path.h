// fast_path.h — register-resident sampler for one row per 512-lane
// workgroup (V <= 53245), the hot path of nis_sample_batch.
//
// HBM is touched once: every lane issues its (up to 26) nontemporal 16-byte
// buffer loads up front.  The row's float4 slots are split evenly over the
// eight waves in whole 64-slot chunks, S per wave (chunk k / lane l of wave
// w holds slot w*S + 64k + l, so every wave owns a contiguous index range),
// and the row then lives in VGPRs (up to 104 logits per lane; 8 waves per
// workgroup leave each wave up to 256 VGPRs).  While the loads stream in,
// each wave adds the masses e = 2^(x*c - R_w) of its elements to Z
// (c = log2(e)/T, R_w a reference from the wave's own first chunk, so no
// workgroup barrier is needed until the stream ends) and keeps the maximum
// of every float4.  The waves' loads are served in wave order, so the first
// half of the waves finishes its stream long before the second half; the
// second half runs at a raised priority.
//
// The top-p cutoff of src/sampler.rs:118-160 is then found without sorting
// the row.  The reference keeps sorted position pos iff
// cum_excl(pos) - q(pos) <= p; that quantity is non-decreasing in pos, so
// the kept set is a prefix of the sorted order and one threshold suffices:
//
// Sparse route (few kept tokens, the common case):
//   1. in the stream, each wave's sample (the float4 maxima of its first 8
//      chunks) gives a threshold th_w, and every float4 holding an element
//      >= th_w is appended to the wave's list, in index order;
//   2. at its stream end the wave compacts its list to single candidates and
//      adds them to two histograms on an absolute grid (whole octaves of x*c
//      and 1/64 octaves, so no wave needs the row max): count and the exact
//      fixed-point sum of 2^frac(x c);
//   3. after the one barrier the stream ends with, every wave on its own
//      finds the cutoff: the deepest octave, then the deepest 1/64-octave
//      bucket, passing a permissive test of sampler.rs:150 (the bucket's
//      upper edge standing in for its largest element), so the cutoff lies
//      in that bucket or the next non-empty one above; x_lo = max th_w is
//      proven safe on the way;
//   4. each wave scans its candidates for the members of those two buckets
//      and the kept mass above them (per 64 index-ordered segments), wave 0
//      ranks the members exactly, and the inverse-CDF walk (sampler.rs:
//      209-216) goes waves -> segments -> the crossing segment's entries.
// Dense route (most tokens kept, or top-p off): a value window around the
// cutoff from a sample, one register pass that adds the mass above the
// window into per-(wave, chunk, lane) cells and lists the window elements,
// a fine histogram of the window, an exact pass over the cutoff bucket, and
// a walk waves -> chunks -> lanes -> elements.
//
// Every step that cannot prove its result (non-finite input, reference
// overflow, a threshold or window that misses the cutoff, list or bucket
// overflow) hands the row to the general path, which recomputes it from HBM.
#pragma once
#include "general_path.h"

namespace nis {

typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
// global-address-space views, so loads are global_load with an SGPR base
typedef const __attribute__((address_space(1))) f4v* gf4p;
typedef const __attribute__((address_space(1))) float* gfp;
typedef int32_t i4v __attribute__((ext_vector_type(4)));

// Raw buffer load of 16 bytes (LLVM's llvm.amdgcn.raw.buffer.load): an
// offset at or past the descriptor's byte count reads zeros and makes no
// memory request.  aux = 2 marks it nontemporal.
__device__ f4v nis_buffer_load_f4(i4v rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4f32");

constexpr int kNch = 26;                      // float4 chunks per lane
constexpr int kFastMaxV = kBlock * 4 * kNch - 3;
constexpr int kSampleBins = 512;              // 32 octaves at 1/16 octave
constexpr float kSampleRes = 16.0f;
constexpr int kBinsPerLane = kSampleBins / 64;
constexpr int kFineBins = 1024;
constexpr int kMaxFinal = 64;
constexpr int kLaneCap = 16;                  // dense route: window entries per lane
constexpr float kMaxT = 60.0f;                // overflow guard for 2^(x*c - R)
constexpr double kFix = 1099511627776.0;      // 2^40 fixed-point mass scale
constexpr uint8_t kKeptBit = 0x80;
// sparse route: each wave takes the float4 maxima of its first kTopS chunks
// as a sample and lists, chunk by chunk as the loads land, the float4s
// reaching the lower edge of the sample's top histogram bins that hold at
// most kTopT of it (bins of 1/kTopRes octave of x*c, from kTopHead octaves
// above the wave's reference down)
constexpr int kTopS = 8;
constexpr uint32_t kTopT = 80;
constexpr int kTopBins = 256;
constexpr float kTopRes = 8.0f;
constexpr float kTopHead = 8.0f;
constexpr int kWaveEnt = 384;                 // listed float4s per wave
constexpr int kWaveCand = 448;                // candidates per wave
// mass histogram of the candidates: kHRes buckets per octave of x*c on an
// absolute grid (bucket floor(64 x c), so every wave agrees on it without
// knowing the row max), kept in a ring of kHB buckets
constexpr int kHB = 2048;

struct DenseShared {
    float cell[kWaves][kNch][64];    // kept mass of each lane's 4 elements per chunk
    float lx[kLaneCap][kBlock];      // lane-private window lists: logit
    uint8_t lp[kLaneCap][kBlock];    //   position 4k+q in the lane, | kKeptBit when kept
    f4v stx[kNch][64];               // the chosen wave's logits, staged for the final lane
    uint32_t cj[kMaxFinal];          // members of the cutoff bucket: row index
    float cx[kMaxFinal];             //   logit
    uint32_t cloc[kMaxFinal];        //   owner thread * kLaneCap + list slot
};
struct SparseShared {
    // per-wave lists (64 slots of slack past each capacity: reads of whole
    // 64-lane groups past a list's end stay inside it)
    union {
        struct {
            f4v ent_x[kWaves][kWaveEnt];         // listed float4s, wave-compacted in index order
            uint16_t ent_pos[kWaves][kWaveEnt];  //   their chunk * 64 + lane
        } l;
        struct {  // members of the cutoff buckets, per wave (the listing is dead by then)
            float gx[kWaves][kMaxFinal];
            uint32_t gi[kWaves][kMaxFinal];
            float ge[kWaves][kMaxFinal];
            uint32_t gj[kWaves][kMaxFinal];  // position in the owner's candidate list
            double seg[kWaves][64];          // kept mass above the cutoff buckets, per list segment
            double mseg[64];                 // the chosen list's kept members, per segment
        } g;
    } u;
    float cx[kWaves][kWaveCand + 64];         // candidates (x >= th_w) in index order: logit
    uint32_t ci[kWaves][kWaveCand + 64];      //   row index
    // [bucket & (kHB-1)]: count << 48 | sum of the members' 2^frac(x c) * 2^24;
    // [kHB + lane]: dummy buckets
    unsigned long long hist[kHB + 64];
    unsigned long long chist[32 + 64];        // the same per octave (ring of 32; dummies)
};

// One 16-byte record per wave, written by the wave's lane 0 and read whole
// by every lane after a barrier (one LDS round trip for all eight).
struct alignas(16) WaveRec {
    double d;
    uint32_t a;
    uint32_t b;
};

// Branches cost about as much as ten VALU instructions here, so the tail
// avoids exec-mask branches: lanes with nothing to store write their own
// slot of `junk`, and masked-off histogram updates go to a dummy bin past
// the end of each histogram.
struct FastShared {
    uint32_t scnt[kSampleBins + 64];        // [kSampleBins + lane]: dummy bins
    uint32_t fcnt[kFineBins + 64];          // [kFineBins + lane]: dummy buckets
    unsigned long long fmass[kFineBins + 64];
    uint32_t fkmax[kFineBins + 64];
    uint32_t fkmin[kFineBins + 64];
    double junk[kBlock];                    // per-lane spare store slot
    union {
        DenseShared d;
        SparseShared s;
    };
    WaveRec t1[kWaves];              // stream end: {Z_w, max_w, R_w}
    WaveRec tc[kWaves];              // listing: {th_w, listed float4s, candidates}
    WaveRec wc[kWaves];              // candidates: {mass, listed float4s, candidates}
    WaveRec wg[kWaves];              // gather: {sure mass, sure count, bucket members}
    uint64_t rng[4];                 // the row's RNG state after its one draw
    uint32_t ncand;
    uint32_t overflow;
    float fa[kWaves];
    float fb[kWaves];
    float fc[kWaves];
    double da[kWaves];
    double db[kWaves];
    int32_t ia[kWaves];
    uint32_t ua[kWaves];
    uint32_t ub[kWaves];
    double wtot[kWaves];
    double ctot[kNch];
    float bf[8];
    double bd[8];
    int32_t bi[8];
    int32_t bi2[kWaves];
    alignas(16) uint32_t ncnt[kWaves];  // candidates per list
};

// Optional per-phase timestamps of each workgroup's wave 0 (profiling
// builds only; compiled out unless NIS_PHASE_TIMING is defined).
#ifdef NIS_PHASE_TIMING
__device__ unsigned long long nis_phase_ts[8192 * 16];
#define NIS_TS(i)                                                                   \
    do {                                                                            \
        if (threadIdx.x == 0) nis_phase_ts[blockIdx.x * 16 + (i)] = wall_clock64(); \
    } while (0)
#else
#define NIS_TS(i) \
    do {          \
    } while (0)
#endif

// Workgroup barrier that orders LDS only, so global loads still in flight
// are not drained by it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Orders one wave's LDS writes before its own later LDS reads of other lanes.
__device__ __forceinline__ void lds_wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Mass of sample bin b (t in (-(b+1)/64, -b/64]) at its centre, for the
// threshold estimates only.
__device__ __forceinline__ float bin_mass(int b) {
    return __builtin_amdgcn_exp2f(-((float)b + 0.5f) * (1.0f / kSampleRes));
}

__device__ __forceinline__ float elem(const f4v& v, int q) {
    return q == 0 ? v.x : (q == 1 ? v.y : (q == 2 ? v.z : v.w));
}
__device__ __forceinline__ uint32_t elemu(const u4v& v, int q) {
    return q == 0 ? v.x : (q == 1 ? v.y : (q == 2 ? v.z : v.w));
}
__device__ __forceinline__ float max4(const f4v& v) {
    return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
}

// Mass of a logit relative to the reference R, in the one form used
// everywhere on this path so that equal logits get bit-equal masses.
__device__ __forceinline__ float mass_of(float x, float c, float R) {
    return __builtin_amdgcn_exp2f(fmaf(x, c, -R));
}

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// LDS stores by the lanes of `mask` only (`mask` must be a subset of the
// active lanes, e.g. a ballot).  exec is narrowed around the stores, so the
// other lanes move no data through the LDS and no branch is taken.  Within
// a wave LDS operations complete in order, and the release fences of the
// barriers wait for them like for any other LDS store.
__device__ __forceinline__ void lds_put_x4_u16(uint64_t mask, uint32_t a, f4v v, uint32_t b,
                                               uint32_t h) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_write_b128 %2, %3\n\t"
        "ds_write_b16 %4, %5\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(v), "v"(b), "v"(h)
        : "memory");
}
__device__ __forceinline__ void lds_put_u32x3(uint64_t mask, uint32_t a, uint32_t va, uint32_t b,
                                              uint32_t vb, uint32_t c, uint32_t vc) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_write_b32 %2, %3\n\t"
        "ds_write_b32 %4, %5\n\t"
        "ds_write_b32 %6, %7\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(va), "v"(b), "v"(vb), "v"(c), "v"(vc)
        : "memory");
}
__device__ __forceinline__ void lds_put_u32x4(uint64_t mask, uint32_t a, uint32_t va, uint32_t b,
                                              uint32_t vb, uint32_t c, uint32_t vc, uint32_t d,
                                              uint32_t vd) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_write_b32 %2, %3\n\t"
        "ds_write_b32 %4, %5\n\t"
        "ds_write_b32 %6, %7\n\t"
        "ds_write_b32 %8, %9\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(va), "v"(b), "v"(vb), "v"(c), "v"(vc), "v"(d), "v"(vd)
        : "memory");
}
// Two 64-bit LDS atomic adds of v by the lanes of `mask` only.
__device__ __forceinline__ void lds_add_u64x2(uint64_t mask, uint32_t a, uint32_t b, uint64_t v) {
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
// one u32 by the wave's lane 0
__device__ __forceinline__ void lds_put_lane0(uint32_t a, uint32_t v) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, 1\n\t"
        "ds_write_b32 %1, %2\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "v"(a), "v"(v)
        : "memory");
}
// a WaveRec by the wave's lane 0
__device__ __forceinline__ void lds_put_rec(uint32_t a, double d, uint32_t x, uint32_t y) {
    const uint64_t db = (uint64_t)__double_as_longlong(d);
    const u4v v = {(uint32_t)db, (uint32_t)(db >> 32), x, y};
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, 1\n\t"
        "ds_write_b128 %1, %2\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "v"(a), "v"(v)
        : "memory");
}
__device__ __forceinline__ void read_recs(const WaveRec* r, double* d, uint32_t* x, uint32_t* y) {
    u4v v[kWaves];
#pragma unroll
    for (int i = 0; i < kWaves; ++i) v[i] = *reinterpret_cast<const u4v*>(&r[i]);
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        d[i] = __longlong_as_double((long long)(((uint64_t)v[i].y << 32) | v[i].x));
        x[i] = v[i].z;
        y[i] = v[i].w;
    }
}
__device__ __forceinline__ void lds_put_u32x2(uint64_t mask, uint32_t a, uint32_t va, uint32_t b,
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

// m * 2^40 as an exact integer, m an f32 mass in [0, 1] (high part m * 2^8,
// low part the rest: both exact in f32).
__device__ __forceinline__ unsigned long long fix40(float m) {
    const float hi = floorf(m * 256.0f);
    const uint32_t lo = (uint32_t)fmaf(-hi, 4294967296.0f, m * 1099511627776.0f);
    return ((unsigned long long)(uint32_t)hi << 32) | lo;
}

// Candidate-histogram bucket of a logit: floor(64 x c), monotone in x.
__device__ __forceinline__ int hbucket(float x, float c) {
    return (int)floorf((x * c) * 64.0f);
}
// Mass of a candidate relative to the integer reference R, in the form the
// candidate histogram sums exactly: 2^frac(x c) scaled by 2^(floor(x c) - R).
__device__ __forceinline__ float canon_mass(float x, float c, int R) {
    const float t = x * c;
    const float fl = floorf(t);
    return ldexpf(__builtin_amdgcn_exp2f(t - fl), (int)fl - R);
}

// Fine-histogram bucket of an element in [x_lo, x_top] (monotone in x).
__device__ __forceinline__ int fine_bucket(float x, float x_lo, float inv_w) {
    return min(max((int)((x - x_lo) * inv_w), 0), kFineBins - 1);
}

// Value of a float4 slot that is not fully inside the row: the few head /
// tail elements come from scalar loads, everything outside the row is -inf.
__device__ __forceinline__ f4v fix_slot(f4v v, int f, int f_lo, int f_hi, int mis, int V, float h0,
                                        float h1, float h2, float t0, float t1, float t2) {
    if (f >= f_lo && f <= f_hi) return v;
    float o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int j = 4 * f + q - mis;
        float y = -INFINITY;
        if (j >= 0 && j < V) {
            if (j < 3) y = (j == 0) ? h0 : (j == 1 ? h1 : h2);
            else y = (j == V - 3) ? t0 : (j == V - 2 ? t1 : t2);
        }
        o[q] = y;
    }
    return f4v{o[0], o[1], o[2], o[3]};
}

// Adds the candidates of the lanes in `ok` to the candidate histograms:
// count << 48 | 2^frac(x c) * 2^24 (LDS atomics by those lanes only).
__device__ __forceinline__ void hist_add(FastShared& sh, float x, float c, bool ok) {
    const float t = x * c;
    const float fl = floorf(t);
    const uint32_t fx = (uint32_t)(__builtin_amdgcn_exp2f(t - fl) * 16777216.0f);
    const uint32_t b = (uint32_t)((int)floorf(t * 64.0f) & (kHB - 1));
    const uint32_t bo = (uint32_t)((int)fl & 31);
    const uint64_t v = (1ull << 48) | (uint64_t)fx;
    lds_add_u64x2(__ballot(ok), lds_addr(&sh.s.hist[0]) + 8 * b, lds_addr(&sh.s.chist[0]) + 8 * bo, v);
}

// Takes wave o's listed float4s [0, ne): every element >= th joins o's
// candidate list (index order; past the capacity the count still grows and
// the row is rejected later).  Lane l takes entries 128 i + 2 l and
// 128 i + 2 l + 1 of step i, and one scan of the per-lane hit counts places
// all hits of the step at once.  Returns the candidate count.  Called by
// the whole wave.
__device__ __forceinline__ uint32_t take_entries(FastShared& sh, int o, uint32_t ne, float th,
                                                 int S, int mis) {
    const int l = lane_id();
    const uint32_t cx0 = lds_addr(&sh.s.cx[o][0]);
    const uint32_t ci0 = lds_addr(&sh.s.ci[o][0]);
    uint32_t nc = 0;
    #pragma unroll 1
    for (uint32_t e0 = 0; e0 < ne; e0 += 128u) {
        const uint32_t e = e0 + 2u * (uint32_t)l;
        const uint32_t ec = min(e, (uint32_t)kWaveEnt - 2u);
        const f4v v0 = sh.s.u.l.ent_x[o][ec];
        const f4v v1 = sh.s.u.l.ent_x[o][ec + 1];
        const uint32_t pp = *reinterpret_cast<const uint32_t*>(&sh.s.u.l.ent_pos[o][ec]);
        uint32_t okm = 0;  // bits 0-3: entry e, bits 4-7: entry e + 1
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            okm |= ((e < ne) & (elem(v0, q) >= th)) ? (1u << q) : 0u;
            okm |= ((e + 1 < ne) & (elem(v1, q) >= th)) ? (16u << q) : 0u;
        }
        const uint32_t cnt = (uint32_t)__popc(okm);
        const uint32_t incl = wscan_u32(cnt);
        const uint32_t base = nc + incl - cnt;
        const int i0 = 4 * (o * S + (int)(pp & 0xFFFFu)) - mis;  // row index of entry e's element 0
        const int i1 = 4 * (o * S + (int)(pp >> 16)) - mis;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const bool ok = (okm >> q) & 1u;
            const uint32_t slot = min(base + (uint32_t)__popc(okm & ((1u << q) - 1u)), (uint32_t)kWaveCand - 1);
            const float x = q < 4 ? elem(v0, q) : elem(v1, q - 4);
            lds_put_u32x2(__ballot(ok), cx0 + 4 * slot, __float_as_uint(x), ci0 + 4 * slot,
                          (uint32_t)((q < 4 ? i0 : i1) + (q & 3)));
        }
        nc += (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    }
    return nc;
}

// Adds wave o's candidates [0, n) to the candidate histograms.
__device__ __forceinline__ void hist_list(FastShared& sh, int o, uint32_t n, float c) {
    const int l = lane_id();
    const int nn = (int)min(n, (uint32_t)kWaveCand);
    #pragma unroll 1
    for (int j0 = 0; j0 < nn; j0 += 64) {
        const int j = j0 + l;
        hist_add(sh, sh.s.cx[o][min(j, kWaveCand - 1)], c, j < nn);
    }
}

__device__ __forceinline__ bool fast_eligible(const RowArgs a, int row) {
    if (a.V < 256 || a.V > kFastMaxV) return false;
    int64_t g0 = 0, g1 = 0;
    if (a.penalty != 1.0f && gen_range(a, row, g0, g1) && g1 > g0)
        return false;
    if (a.temperature <= 0.0f) return true;
    if (a.top_k > 0 && a.top_k < (uint64_t)a.V) return false;
    if (a.top_p <= 0.0f) return false;
    return true;
}

// Returns NIS_REJECT_NONE when the row is done, else (uniformly across the
// workgroup) why it must be recomputed by the general path; nothing has been
// written then.
__device__ __forceinline__ uint32_t fast_row(const RowArgs a, const int row, FastShared& sh) {
    const int tid = threadIdx.x, l = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());  // wave-uniform
    const int V = (int)a.V;
    const gfp rowp = (gfp)(a.logits + (int64_t)row * a.ld);
    const int mis = (int)(((uintptr_t)rowp >> 2) & 3);  // elements before the row in its 16 B block
    const gf4p base = (gf4p)(rowp - mis);
    const int f_lo = mis ? 1 : 0;          // first float4 slot lying fully inside the row
    const int f_hi = (V + mis - 4) >> 2;   // last one
    // The slots touching the row are split evenly over the waves in whole
    // chunks: wave w owns slots [w*S, w*S + S).  Kw of its chunks reach into
    // the row; the stream processes Kp of them (at least the sample chunks).
    // The loads of chunks past Kw read nothing (out-of-range buffer offsets)
    // and those chunks hold -inf.
    const int nsl = (V + mis + 3) >> 2;
    const int S = 64 * ((nsl + 64 * kWaves - 1) / (64 * kWaves));
    const int Kw = min(max((nsl - w * S + 63) >> 6, 0), S >> 6);
    const int Kp = max(Kw, kTopS);
    const int slot0 = w * S + l;
    const bool sampling = a.temperature > 0.0f;

    NIS_TS(0);
    // the (at most 3 + 3) elements of the partial head / tail slots, first:
    // the waves holding such slots need them before their first chunk
    const float h0 = rowp[0], h1 = rowp[1], h2 = rowp[2];
    const float t0 = rowp[V - 3], t1 = rowp[V - 2], t2 = rowp[V - 1];
    __builtin_amdgcn_sched_barrier(0);
    // buffer descriptor over the row's whole float4 slots [0, f_hi]: slots
    // past the row read zeros (fixed below); the partial head slot is
    // redirected to f_lo so nothing before the row is touched
    const uint64_t bptr = (uint64_t)(uintptr_t)base;
    const i4v rsrc = {(int32_t)(uint32_t)bptr, (int32_t)(uint32_t)((bptr >> 32) & 0xFFFFu),
                      16 * (f_hi + 1), 0x00020000};
    f4v xv[kNch];
#pragma unroll
    for (int k = 0; k < kNch; ++k) {
        const int f = slot0 + k * 64;
        const int off = (k < Kw) ? 16 * max(f, f_lo) : 0x7FFFFFF0;
        xv[k] = nis_buffer_load_f4(rsrc, off, 0, 2);
        __builtin_amdgcn_sched_barrier(0);  // keep chunk order = issue order
    }
    // the row's RNG state (sampler.rs:209 draws from it once), loaded behind
    // the logits so that the draw does not wait for it later.  Greedy calls
    // may pass no states (the C ABI allows that only for temperature <= 0):
    // the load then reads the row's first whole float4 slots instead, and
    // the value is never used.
    typedef const __attribute__((address_space(1))) uint64_t* gu64p;
    const gu64p rng_src = a.rng ? (gu64p)(a.rng + 4 * (int64_t)row) : (gu64p)(rowp - mis + 4 * f_lo);
    const uint64_t rsv = rng_src[l & 3];

    // LDS store by the lanes where `cond` holds; the other lanes write their
    // own spare slot, so no exec-mask branch is needed
#define NIS_PUT(cond, ref, val)                                                             \
    do {                                                                                    \
        auto* nis_dst_ = (cond) ? &(ref) : reinterpret_cast<decltype(&(ref))>(&sh.junk[tid]); \
        *nis_dst_ = (val);                                                                  \
    } while (0)

    // LDS set-up while the loads are in flight
    static_assert(kSampleBins == kBlock, "one sample bin per lane to clear");
    sh.scnt[tid] = 0u;
#pragma unroll
    for (int j = 0; j < kFineBins / kBlock; ++j) {
        sh.fcnt[tid + j * kBlock] = 0u;
        sh.fmass[tid + j * kBlock] = 0ull;
        sh.fkmax[tid + j * kBlock] = 0u;
        sh.fkmin[tid + j * kBlock] = 0xFFFFFFFFu;
    }
    NIS_PUT(tid == 0, sh.ncand, 0u);
    NIS_PUT(tid == 0, sh.overflow, 0u);
    // this wave's histogram of float4 maxima (in its own candidate row, which
    // is written only after the histogram is read)
    static_assert(kTopBins == 4 * 64 && kTopBins <= kWaveCand + 64, "4 bins per lane, inside a row");
    *reinterpret_cast<u4v*>(reinterpret_cast<uint32_t*>(&sh.s.cx[w][0]) + 4 * l) = u4v{0u, 0u, 0u, 0u};

    // slots not fully inside the row get their exact values or -inf; only
    // the one or two waves holding such slots take the (wave-uniform) branch.
    // slot0x is an opaque copy of slot0: the per-chunk slot numbers are then
    // recomputed where needed instead of being kept live from the loads.
    int slot0x = slot0;
    asm volatile("" : "+v"(slot0x));
#define NIS_FIX(k)                                                                          \
    do {                                                                                    \
        const int fb0 = w * S + (k) * 64;                                                   \
        if (fb0 < f_lo || fb0 + 63 > f_hi)                                                  \
            xv[k] = fix_slot(xv[k], slot0x + (k) * 64, f_lo, f_hi, mis, V, h0, h1, h2, t0, t1, t2); \
    } while (0)
#define NIS_INDEX(k, q) (4 * (slot0x + 64 * (k)) + (q) - mis)
    // does this wave hold any slot not fully inside the row?  Only such
    // waves run the per-chunk checks (each one is a branch).
    const bool edge_wave = (w * S < f_lo) || (w * S + 64 * Kw - 1 > f_hi);

    // ------------------------------------------------------------------
    // greedy (sampler.rs:172-181): first index of the maximum; NaN is
    // skipped by the strict `>`, except that a NaN at index 0 wins.
    if (!sampling) {
        float best = -INFINITY;
        int bidx = INT_MAX;
#define NIS_GREEDY(FIX)                                      \
    _Pragma("unroll") for (int k = 0; k < kNch; ++k) if (k < Kw) { \
        if (FIX) NIS_FIX(k);                                 \
        _Pragma("unroll") for (int q = 0; q < 4; ++q) {     \
            const float x = elem(xv[k], q);                  \
            if (x > best) {                                  \
                best = x;                                    \
                bidx = NIS_INDEX(k, q);                      \
            }                                                \
        }                                                    \
    }
        if (edge_wave) {
            NIS_GREEDY(true)
        } else {
            NIS_GREEDY(false)
        }
#undef NIS_GREEDY
        // wave max, then its lowest index (lanes interleave indices chunk by
        // chunk, so the lowest lane holding the max need not hold the lowest index)
        // (DPP max of the negated index; indices < 2^24 are exact in float)
        const float wb = wmax_f32(best);
        const float nwi = wmax_f32((best == wb && bidx != INT_MAX) ? -(float)bidx : -INFINITY);
        const int wi = (nwi > -INFINITY) ? (int)(-nwi) : INT_MAX;
        NIS_PUT(l == 0, sh.fa[w], wb);
        NIS_PUT(l == 0, sh.ia[w], wi);
        lds_barrier();
        if (tid == 0) {
            float b = sh.fa[0];
            int bi = sh.ia[0];
            for (int i = 1; i < kWaves; ++i)
                if (sh.fa[i] > b || (sh.fa[i] == b && sh.ia[i] < bi)) {
                    b = sh.fa[i];
                    bi = sh.ia[i];
                }
            const uint32_t tok = (h0 != h0 || bi == INT_MAX) ? 0u : (uint32_t)bi;
            write_row_result(a, row, tok, NIS_PATH_GREEDY, 0.0, 0.0, 0.0, -1.0, 0.0, 0, 1);
        }
        return NIS_REJECT_NONE;
    }

    // ------------------------------------------------------------------
    const double temp = fmax((double)a.temperature, 1e-6);  // sampler.rs:183
    const float c = (float)(1.4426950408889634 / temp);     // log2(e) / T
    const float p = a.top_p;
    const bool topp = p < 1.0f;  // p <= 0 is excluded by fast_eligible

    // The candidate histograms are cleared by the first half of the waves
    // (whose loads were issued first and land first); the second half runs
    // at a raised priority, ahead of the first half's work on the same
    // SIMDs once its data arrives.
    if (w >= kWaves / 2) {
        __builtin_amdgcn_s_setprio(2);
    } else {
        for (int i = tid; i < kHB + 64; i += kBlock / 2) sh.s.hist[i] = 0ull;
        if (tid < 32 + 64) sh.s.chist[tid] = 0ull;
    }

    // wave-local reference from the wave's first chunk
    if (Kw == 0)
        xv[0] = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    else if (edge_wave)
        NIS_FIX(0);
    const float m0 = wmax_f32(max4(xv[0]));
    const float Rw = (m0 > -INFINITY && fabsf(m0 * c) < 1e30f) ? ceilf(m0 * c) : 0.0f;
    const float RwH = Rw + kTopHead;

    // masses and Z, chunk by chunk as the loads land.  cz / Rz are opaque
    // copies of c / Rw: without them the compiler merges these masses with
    // identical later ones and keeps all 104 of them live.
    //
    // Sparse top-p candidates are listed in the same pass (the loads of later
    // chunks are still in flight meanwhile): a count histogram of the float4
    // maxima of the first kTopS chunks (fire-and-forget LDS atomics, 1/8-
    // octave bins from kTopHead octaves above the wave's reference) gives
    // th_w, the lower edge of its top bins holding at most kTopT of them;
    // every float4 holding an element >= th_w is then appended to the wave's
    // list (index order, only the hit lanes store; past the capacity they
    // all write the last slot and the overflow is caught after the stream).
    // x_lo = max over the waves of th_w is a threshold at and above which
    // every element is listed; th_w = +inf when no bin fits, and without
    // top-p.
    double z = 0.0;
    float mx = -INFINITY;
    float mx4[kNch];
    float cz = c, Rz = Rw;
    asm volatile("" : "+v"(cz), "+v"(Rz));
    uint32_t* const whist = reinterpret_cast<uint32_t*>(&sh.s.cx[w][0]);
    const uint32_t ent_x0 = lds_addr(&sh.s.u.l.ent_x[w][0]);
    const uint32_t ent_p0 = lds_addr(&sh.s.u.l.ent_pos[w][0]);
    float thw = INFINITY;
    uint32_t nw = 0;
#define NIS_LIST(k)                                                                      \
    {                                                                                    \
        const uint64_t mk = __ballot(mx4[k] >= thw);                                     \
        const uint32_t slot = min(nw + lane_rank(mk), (uint32_t)kWaveEnt - 1);           \
        lds_put_x4_u16(mk, ent_x0 + 16 * slot, xv[k], ent_p0 + 2 * slot, (uint32_t)((k) * 64 + l)); \
        nw += (uint32_t)__popcll(mk);                                                    \
    }
#define NIS_STREAM(FIX)                                                                 \
    _Pragma("unroll") for (int k = 0; k < kNch; ++k) if (k >= Kp) {                     \
        xv[k] = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};                        \
    } else {                                                                            \
        if (k >= Kw) xv[k] = f4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};           \
        else if (FIX && k > 0) NIS_FIX(k);                                              \
        const f4v x = xv[k];                                                            \
        f4v e;                                                                          \
        e.x = mass_of(x.x, cz, Rz);                                                     \
        e.y = mass_of(x.y, cz, Rz);                                                     \
        e.z = mass_of(x.z, cz, Rz);                                                     \
        e.w = mass_of(x.w, cz, Rz);                                                     \
        z += (double)((e.x + e.y) + (e.z + e.w));                                       \
        mx4[k] = max4(x);                                                               \
        mx = fmaxf(mx, mx4[k]);                                                         \
        if (k < kTopS) {                                                                \
            const float tb = floorf((RwH - mx4[k] * cz) * kTopRes); /* -inf -> +inf */   \
            atomicAdd(&whist[(uint32_t)fminf(fmaxf(tb, 0.0f), (float)(kTopBins - 1))], 1u); \
        }                                                                               \
        if (k == kTopS - 1) {                                                           \
            lds_wave_fence();                                                           \
            const u4v hc = *reinterpret_cast<const u4v*>(&whist[4 * l]); /* bins 4l.. */ \
            const uint32_t hs = hc.x + hc.y + hc.z + hc.w;                              \
            const uint32_t hi = wscan_u32(hs);                                          \
            const uint32_t c0 = hi - hs + hc.x, c1 = c0 + hc.y, c2 = c1 + hc.z, c3 = c2 + hc.w; \
            const uint32_t nok = (uint32_t)(c0 <= kTopT) + (uint32_t)(c1 <= kTopT) +    \
                                 (uint32_t)(c2 <= kTopT) + (uint32_t)(c3 <= kTopT);     \
            const int bw = (int)wsum_u32(nok) - 1; /* the last bin whose count fits */  \
            /* mass of the sampled maxima below the threshold (lower bound), and */    \
            /* of all sampled elements (upper bound: 4x the maxima): when the */        \
            /* first already exceeds what top-p may drop, the row is not sparse */     \
            const float e0 = __builtin_amdgcn_exp2f(-(float)(4 * l) * (1.0f / kTopRes)); \
            const float mq0 = (float)hc.x * e0, mq1 = (float)hc.y * e0 * 0.917004043f;   \
            const float mq2 = (float)hc.z * e0 * 0.840896415f, mq3 = (float)hc.w * e0 * 0.771105413f; \
            const float mlo = ((4 * l + 0 > bw) ? (float)hc.x * e0 * 0.917004043f : 0.0f) + \
                              ((4 * l + 1 > bw) ? (float)hc.y * e0 * 0.840896415f : 0.0f) + \
                              ((4 * l + 2 > bw) ? (float)hc.z * e0 * 0.771105413f : 0.0f) + \
                              ((4 * l + 3 > bw) ? (float)hc.w * e0 * 0.707106781f : 0.0f); \
            const bool flat = wsum_f32(mlo) > 4.0f * (1.0f - p) * wsum_f32(mq0 + mq1 + mq2 + mq3); \
            thw = (!topp || bw < 0 || flat) ? INFINITY : (RwH - (float)(bw + 1) * (1.0f / kTopRes)) / c; \
            _Pragma("unroll") for (int j = 0; j < kTopS; ++j) NIS_LIST(j)               \
        }                                                                               \
        if (k >= kTopS) NIS_LIST(k)                                                     \
    }
    if (edge_wave) {
        NIS_STREAM(true)
    } else {
        NIS_STREAM(false)
    }
#undef NIS_STREAM
#undef NIS_LIST
    NIS_TS(1);

    // ---- stream end: this wave's totals, threshold and list length -------
    mx = wmax_f32(mx);
    z = wsum_f64(z);
    lds_put_rec(lds_addr(&sh.t1[w]), z, __float_as_uint(mx), __float_as_uint(Rw));
    lds_put_rec(lds_addr(&sh.tc[w]), (double)thw, nw, 0u);

    // ---- candidates: every wave takes its own list once its stream ends.
    // One barrier orders the clearing of the histograms before any addition:
    // the first half compacts its list before it (its data came first) and
    // adds to the histograms after it; the second half takes the barrier at
    // its stream end, where the first half is already waiting.
    if (w < kWaves / 2) {
        const uint32_t nco = topp ? take_entries(sh, w, min(nw, (uint32_t)kWaveEnt), thw, S, mis) : 0u;
        lds_barrier();
        if (topp) {
            hist_list(sh, w, nco, c);
            lds_put_lane0(lds_addr(&sh.ncnt[w]), nco);
        }
    } else {
        lds_barrier();
        if (topp) {
            const uint32_t nco = take_entries(sh, w, min(nw, (uint32_t)kWaveEnt), thw, S, mis);
            hist_list(sh, w, nco, c);
            lds_put_lane0(lds_addr(&sh.ncnt[w]), nco);
        }
    }
    // sampler.rs:209: the row's single RNG advance, drawn here by wave 0
    // into LDS; written back to memory only when the row completes on this
    // path.
    if (w == 0) {
        uint64_t st[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            st[j] = ((uint64_t)bcast_u32((uint32_t)(rsv >> 32), j) << 32) | bcast_u32((uint32_t)rsv, j);
        const double u0 = rng_next_f64(st);
        NIS_PUT(l == 0, sh.bd[1], u0);
        NIS_PUT(l == 1, sh.rng[0], st[0]);
        NIS_PUT(l == 2, sh.rng[1], st[1]);
        NIS_PUT(l == 3, sh.rng[2], st[2]);
        NIS_PUT(l == 4, sh.rng[3], st[3]);
    }

    NIS_TS(2);

    // ---- T1: row max, reference R, Z ---------------------------------------
    lds_barrier();
    double zw[kWaves];
    uint32_t mxw[kWaves], rww[kWaves];
    read_recs(sh.t1, zw, mxw, rww);
    float M = __uint_as_float(mxw[0]);
#pragma unroll
    for (int i = 1; i < kWaves; ++i) M = fmaxf(M, __uint_as_float(mxw[i]));
    const float R = (M > -INFINITY && fabsf(M * c) < 1e30f) ? ceilf(M * c) : 0.0f;
    double ZR = 0.0;
    bool range_ok = true;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        // each wave's masses were taken against its own reference; a wave
        // whose reference sits far below the row max may have overflowed
        const float rw = __uint_as_float(rww[i]);
        range_ok = range_ok & (fmaf(M, c, -rw) <= kMaxT);
        ZR += ldexp(zw[i], (int)(rw - R));  // exact power-of-two rescale
    }
    const float tM = fmaf(M, c, -R);
    // NaN / inf input, an empty row, or a reference too far below the max
    if (!(M > -INFINITY) || !(M < INFINITY) || !(ZR > 0.0) || !(ZR < INFINITY) || !range_ok ||
        !(fabsf(M * c) < 1e30f))
        return NIS_REJECT_NONFINITE;
    // R-units -> units of the max element's mass (tM in (-1, 0])
    const double rho = (double)__builtin_amdgcn_exp2f(-tM);
    const double pZ = (double)p * ZR * rho;
    const double pZR = (double)p * ZR;

    uint32_t reject = NIS_REJECT_NONE;  // reason of a failed sparse attempt
    if (topp) {
        double thv[kWaves];
        uint32_t nwv[kWaves], unused[kWaves];
        read_recs(sh.tc, thv, nwv, unused);
        const u4v nca = *reinterpret_cast<const u4v*>(&sh.ncnt[0]);
        const u4v ncb = *reinterpret_cast<const u4v*>(&sh.ncnt[4]);
        uint32_t ncv[kWaves];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            ncv[q] = elemu(nca, q);
            ncv[q + 4] = elemu(ncb, q);
        }
        float x_lo = -INFINITY, th_min = INFINITY;
        uint32_t nwmax = 0, ncmax = 0;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) {
            x_lo = fmaxf(x_lo, (float)thv[i]);
            th_min = fminf(th_min, (float)thv[i]);
            nwmax = max(nwmax, nwv[i]);
            ncmax = max(ncmax, ncv[i]);
        }
        NIS_TS(3);
        // the histogram rings must hold every candidate without aliasing, and
        // bucket numbers must fit an int
        const bool fits = (x_lo < INFINITY) & (x_lo <= M) & (fabsf(M * c) < 1e6f) &
                          (fabsf(th_min * c) < 1e6f);
        const int bM = fits ? hbucket(M, c) : 0;
        const int blo = fits ? hbucket(x_lo, c) : 0;
        const int bmn = fits ? hbucket(th_min, c) : 0;
        reject = NIS_REJECT_CAPACITY;
        if (fits & (nwmax <= (uint32_t)kWaveEnt) & (ncmax <= (uint32_t)kWaveCand) &
            (bM - bmn < kHB) & ((bM >> 6) - (bmn >> 6) < 32)) {
            const int Ri = (int)R;
            // ---- S4: the cutoff, located by every wave on its own (no
            // barrier).  sampler.rs:150 is tested on each bucket's largest
            // element with the bucket's upper edge standing in for it: a
            // permissive test, so the cutoff lies in the lowest passing
            // non-empty bucket or in the next non-empty one above it.
            // Octaves first (lane l: octave oM - l), then the 1/64-octave
            // buckets of the two candidate octaves.  Everything above x_lo's
            // bucket is complete in the histograms.
            const int oM = bM >> 6, olo = blo >> 6;
            const int nco = oM - olo;  // octaves above x_lo's, < 32
            const int oc = oM - l;
            const bool cin = l <= nco;
            const unsigned long long cv = cin ? sh.s.chist[oc & 31] : 0ull;
            const double cm = ldexp((double)(cv & 0xFFFFFFFFFFFFull), oc - Ri - 24);
            const double cG = wscan_f64(cm) - cm;  // mass of the octaves above
            const double cup = ldexp(1.0001, oc + 1 - Ri);
            const bool cne = cin & ((cv >> 48) != 0ull);
            const uint64_t cpass = __ballot(cne & (cG - cup <= pZR));
            const uint64_t cnem = __ballot(cne);
            // octave x_lo lies in: everything up to its top is removed
            const bool clo_ok = __builtin_amdgcn_readlane((int)(cG - cup > pZR), nco) != 0;
            const int lp = cpass ? 63 - __clzll((long long)cpass) : -1;  // deepest passing octave
            const uint64_t above_p = (lp > 0) ? (cnem & ((1ull << lp) - 1ull)) : 0ull;
            const int la = above_p ? 63 - __clzll((long long)above_p) : -1;
            const int Cp = oM - lp, Ca = (la >= 0) ? oM - la : Cp;
            const double Gcp = bcast_f64(cG, max(lp, 0));
            const double Gca = bcast_f64(cG, max(la, 0));
            // fine level: lane l holds bucket 64 C + 63 - l of C = Cp and of C = Ca
            const int bp_l = 64 * Cp + 63 - l, ba_l = 64 * Ca + 63 - l;
            const unsigned long long fpv = sh.s.hist[bp_l & (kHB - 1)];
            const unsigned long long fav = sh.s.hist[ba_l & (kHB - 1)];
            const double fpm = ldexp((double)(fpv & 0xFFFFFFFFFFFFull), Cp - Ri - 24);
            const double fam = ldexp((double)(fav & 0xFFFFFFFFFFFFull), Ca - Ri - 24);
            const double Gp_l = Gcp + (wscan_f64(fpm) - fpm);  // mass above each bucket
            const double Ga_l = Gca + (wscan_f64(fam) - fam);
            const float fe = __builtin_amdgcn_exp2f((float)(63 - l + 1) * (1.0f / 64.0f)) * 1.0001f;
            const double eup_p = ldexp((double)fe, Cp - Ri), eup_a = ldexp((double)fe, Ca - Ri);
            const bool pne = ((fpv >> 48) != 0ull) & (bp_l > blo);
            const bool ane = ((fav >> 48) != 0ull) & (la >= 0);
            const uint64_t ppass = __ballot(pne & (Gp_l - eup_p <= pZR));
            const uint64_t apass = __ballot(ane & (Ga_l - eup_a <= pZR));
            const uint64_t pnem = __ballot(pne), anem = __ballot(ane);
            // the deepest passing bucket b_p, and the next non-empty one above
            int b_p, b_a, lgp, lga;  // lgp / lga: lanes whose running masses give G
            bool gin_p, gin_a;       // ... taken in the Cp (true) or Ca (false) octave
            if (ppass) {
                const int lb = 63 - __clzll((long long)ppass);
                b_p = 64 * Cp + 63 - lb;
                lgp = lb;
                gin_p = true;
                const uint64_t up = pnem & ((1ull << lb) - 1ull);
                if (up) {
                    lga = 63 - __clzll((long long)up);
                    b_a = 64 * Cp + 63 - lga;
                    gin_a = true;
                } else if (anem) {
                    lga = 63 - __clzll((long long)anem);
                    b_a = 64 * Ca + 63 - lga;
                    gin_a = false;
                } else {
                    b_a = b_p;
                    lga = lgp;
                    gin_a = true;
                }
            } else {
                const int lb = apass ? 63 - __clzll((long long)apass) : 0;
                b_p = 64 * Ca + 63 - lb;
                lgp = lb;
                gin_p = false;
                const uint64_t up = anem & ((1ull << lb) - 1ull);
                lga = up ? 63 - __clzll((long long)up) : lb;
                b_a = 64 * Ca + 63 - lga;
                gin_a = false;
            }
            const double gtop = bcast_f64(gin_a ? Gp_l : Ga_l, lga);  // mass above b_a
            // x_lo's bucket and everything below it is removed
            const int llo = 64 * Cp + 63 - blo;
            const bool flo_ok = __builtin_amdgcn_readlane(
                                    (int)(Gp_l - ldexp((double)fe, Cp - Ri) > pZR), min(max(llo, 0), 63)) != 0;
            const bool lo_ok = (Cp > olo) ? clo_ok : flo_ok;
            NIS_TS(4);
            if (!lo_ok || lp < 0 || !(ppass | apass)) {
                reject = NIS_REJECT_WINDOW;  // the cutoff may lie at or below x_lo
            } else {
                // ---- each wave over its own candidates: the members of the
                // two buckets, and the kept mass of everything above them, in
                // 64 index-ordered segments ---------------------------------
                const int ncw = (int)min(ncv[w], (uint32_t)kWaveCand);
                const int sg = (ncw + 63) >> 6;
                constexpr int kSeg = (kWaveCand + 63) / 64;
                float xs[kSeg];
                uint32_t is[kSeg];
#pragma unroll
                for (int i = 0; i < kSeg; ++i) {
                    const int jc = min(l * sg + i, kWaveCand - 1);
                    xs[i] = (i < sg) ? sh.s.cx[w][jc] : -INFINITY;
                    is[i] = (i < sg) ? sh.s.ci[w][jc] : 0u;
                }
                double ssum = 0.0;
                uint32_t scount = 0, memm = 0;
                float es[kSeg];
#pragma unroll
                for (int i = 0; i < kSeg; ++i) {
                    es[i] = 0.0f;
                    if (i < sg) {  // (wave-uniform)
                        const int j = l * sg + i;
                        const bool v = j < ncw;
                        const int b = hbucket(xs[i], c);
                        es[i] = canon_mass(xs[i], c, Ri);
                        const bool sure = v & (b > b_a);
                        ssum += sure ? (double)es[i] : 0.0;
                        scount += sure ? 1u : 0u;
                        memm |= (v & ((b == b_p) | (b == b_a))) ? (1u << i) : 0u;
                    }
                }
                sh.s.u.g.seg[w][l] = ssum;
                const uint32_t nml = (uint32_t)__popc(memm);
                const uint32_t mincl = wscan_u32(nml);
                const uint32_t nm = (uint32_t)__builtin_amdgcn_readlane((int)mincl, 63);
                const uint32_t gx0 = lds_addr(&sh.s.u.g.gx[w][0]);
                const uint32_t gi0 = lds_addr(&sh.s.u.g.gi[w][0]);
                const uint32_t ge0 = lds_addr(&sh.s.u.g.ge[w][0]);
                const uint32_t gj0 = lds_addr(&sh.s.u.g.gj[w][0]);
#pragma unroll
                for (int i = 0; i < kSeg; ++i) {
                    const uint32_t sc =
                        min(mincl - nml + (uint32_t)__popc(memm & ((1u << i) - 1u)), (uint32_t)kMaxFinal - 1);
                    lds_put_u32x4(__ballot((memm >> i) & 1u), gx0 + 4 * sc, __float_as_uint(xs[i]),
                                  gi0 + 4 * sc, is[i], ge0 + 4 * sc, __float_as_uint(es[i]), gj0 + 4 * sc,
                                  (uint32_t)(l * sg + i));
                }
                const double sw = wsum_f64(ssum);
                const uint32_t sn = wsum_u32(scount);
                lds_put_rec(lds_addr(&sh.wg[w]), sw, sn, nm);
                lds_barrier();
                NIS_TS(5);
                double sww[kWaves];
                uint32_t snw[kWaves], nmw[kWaves];
                read_recs(sh.wg, sww, snw, nmw);
                uint32_t nmtot = 0;
#pragma unroll
                for (int i = 0; i < kWaves; ++i) nmtot += nmw[i];
                if (nmtot > (uint32_t)kMaxFinal) {
                    reject = NIS_REJECT_BUCKET;
                } else {
                    // ---- wave 0 alone from here: the exact rule among the
                    // members, the draw, and the walk ----------------------------
                    if (w != 0) return NIS_REJECT_NONE;
                    const int n = (int)nmtot;
                    const bool valid = l < n;
                    // member l of the waves' lists taken in wave order
                    int mwv = 0;
                    uint32_t mbase = 0, acc = 0;
#pragma unroll
                    for (int i = 0; i < kWaves; ++i) {
                        const bool here = (uint32_t)l >= acc;
                        mwv = here ? i : mwv;
                        mbase = here ? acc : mbase;
                        acc += nmw[i];
                    }
                    const int mj = min(l - (int)mbase, kMaxFinal - 1);  // in bounds for every lane
                    const float gxv = sh.s.u.g.gx[mwv][mj];
                    const uint32_t giv = sh.s.u.g.gi[mwv][mj];
                    const float gev = sh.s.u.g.ge[mwv][mj];
                    const uint32_t gjv = sh.s.u.g.gj[mwv][mj];
                    sh.s.u.g.mseg[l] = 0.0;
                    const float xm = valid ? gxv : -INFINITY;
                    const uint32_t im = valid ? giv : 0xFFFFFFFFu;
                    const float em = valid ? gev : 0.0f;
                    // sort key: value descending, then index ascending
                    const uint64_t km = ((uint64_t)key32(xm) << 32) | (uint64_t)(~im);
                    // mass of the members ahead of this one in the reference's
                    // stable descending order
                    double pre = 0.0;
                    #pragma unroll 1
                    for (int j0 = 0; j0 < n; j0 += 4) {
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const int j = min(j0 + u, 63);
                            const uint64_t kj = ((uint64_t)bcast_u32((uint32_t)(km >> 32), j) << 32) |
                                                bcast_u32((uint32_t)km, j);
                            const float ej = bcast_f32(em, j);
                            pre += ((j0 + u < n) & (kj > km)) ? (double)ej : 0.0;
                        }
                    }
                    const bool kept = valid & (gtop + pre - (double)em <= pZR);
                    // the last kept member: smallest value, then largest index
                    // (DPP maxima; indices < 2^24 are exact in float)
                    const float xcut = -wmax_f32(kept ? -xm : -INFINITY);
                    const float icut = wmax_f32((kept & (xm == xcut)) ? (float)im : -1.0f);
                    const uint32_t kc = key32(xcut), ic = (uint32_t)icut;
                    // per-wave kept mass and count (lanes 0..7): the wave's sure
                    // part plus its kept members, which sit in lanes
                    // [start_w, start_w + nm_w) in wave order
                    const double kin = wscan_f64(kept ? (double)em : 0.0);
                    const uint32_t kcn = wscan_u32(kept ? 1u : 0u);
                    const int li = min(l, kWaves - 1);
                    uint32_t st = 0, nmi = nmw[0];
                    double T = sww[0];
                    uint32_t TN = snw[0];
#pragma unroll
                    for (int i = 1; i < kWaves; ++i) {
                        st += (i <= li) ? nmw[i - 1] : 0u;
                        nmi = (li == i) ? nmw[i] : nmi;
                        T = (li == i) ? sww[i] : T;
                        TN = (li == i) ? snw[i] : TN;
                    }
                    const int hi = (int)(st + nmi) - 1, lo = (int)st - 1;
                    const double khi = __shfl(kin, max(hi, 0)), klo = __shfl(kin, max(lo, 0));
                    const uint32_t chi = __shfl(kcn, max(hi, 0)), clo = __shfl(kcn, max(lo, 0));
                    T += (nmi != 0u) ? (khi - ((lo >= 0) ? klo : 0.0)) : 0.0;
                    TN += (nmi != 0u) ? (chi - ((lo >= 0) ? clo : 0u)) : 0u;
                    T = (l < kWaves) ? T : 0.0;
                    TN = (l < kWaves) ? TN : 0u;
                    const double Tincl = wscan_f64(T);
                    const double zk = bcast_f64(Tincl, 63);
                    const uint32_t kept_total = wsum_u32(TN);
                    const double u = sh.bd[1];  // the draw (sampler.rs:209), made before T1
                    const double r = u * zk;
                    // the first wave whose running total reaches r (and has
                    // mass); rounding: the last wave with mass
                    const uint64_t hw = __ballot((l < kWaves) & (T > 0.0) & (Tincl >= r));
                    const uint64_t nzw = __ballot((l < kWaves) & (T > 0.0));
                    const int wsel = hw ? (__ffsll((long long)hw) - 1) : (63 - __clzll((long long)nzw));
                    const double run = bcast_f64(Tincl - T, wsel);
                    int ncsel = (int)min(ncv[0], (uint32_t)kWaveCand);
#pragma unroll
                    for (int i = 1; i < kWaves; ++i)
                        ncsel = (i == wsel) ? (int)min(ncv[i], (uint32_t)kWaveCand) : ncsel;
                    const int sgs = (ncsel + 63) >> 6;
                    NIS_TS(6);
                    // ---- S7: the walk (sampler.rs:209-216) over the chosen
                    // wave's candidates: the segment whose running total
                    // reaches r (sure mass from the scan plus the kept members,
                    // whose masses within the two buckets add exactly in any
                    // order), then that segment's entries, one per lane
                    if (kept & (mwv == wsel)) atomicAdd(&sh.s.u.g.mseg[min((int)gjv / max(sgs, 1), 63)], (double)em);
                    const double lsum = sh.s.u.g.seg[wsel][l] + sh.s.u.g.mseg[l];
                    const double sincl = wscan_f64(lsum);
                    const uint64_t hitl = __ballot((run + sincl >= r) & (lsum > 0.0));
                    const uint64_t nzl = __ballot(lsum > 0.0);
                    const int Ls = hitl ? (__ffsll((long long)hitl) - 1) : max(63 - __clzll((long long)nzl), 0);
                    const double run2 = bcast_f64(run + sincl - lsum, Ls);
                    const int je = Ls * sgs + l;
                    const bool ve = (l < sgs) & (je < ncsel);
                    const float xe = sh.s.cx[wsel][min(je, kWaveCand - 1)];
                    const uint32_t ie = sh.s.ci[wsel][min(je, kWaveCand - 1)];
                    const uint32_t ke = key32(xe);
                    const bool kj = ve & ((ke > kc) | ((ke == kc) & (ie <= ic)));
                    const float ee = kj ? canon_mass(xe, c, Ri) : 0.0f;
                    const double pe = wscan_f64((double)ee);
                    const uint64_t hite = __ballot(kj & (run2 + pe >= r));
                    const uint64_t kje = __ballot(kj);
                    // rounding: the segment's last kept token
                    const int Le = hite ? (__ffsll((long long)hite) - 1) : max(63 - __clzll((long long)kje), 0);
                    if (l == Le) {
                        int tok = (int)ie;
                        bool tkept = true;
                        if (u == 0.0) {  // r == 0 stops the reference's walk at index 0
                            tok = 0;
                            tkept = false;
                        }
                        const double zkM = zk * rho;
                        const double prob = tkept ? (double)ee / zk : 0.0;
                        write_row_result(a, row, (uint32_t)tok, NIS_PATH_DRAW, (double)M / temp,
                                         zkM, ZR * rho, u, prob, (uint64_t)kept_total, 1);
                    }
                    if (l == 0) {
                        uint64_t* sp = a.rng + 4 * (int64_t)row;
                        sp[0] = sh.rng[0];
                        sp[1] = sh.rng[1];
                        sp[2] = sh.rng[2];
                        sp[3] = sh.rng[3];
                    }
                    NIS_TS(9);
                    return NIS_REJECT_NONE;
                }
            }
        }
        // the sparse route gave up: the dense route starts from clean buckets
        // and a count histogram of chunks 0 and 1 (its sample), 1/16-octave
        // bins below R
        __syncthreads();
        for (int i = tid; i < kFineBins; i += kBlock) {
            sh.fcnt[i] = 0u;
            sh.fmass[i] = 0ull;
            sh.fkmax[i] = 0u;
            sh.fkmin[i] = 0xFFFFFFFFu;
        }
        if (tid == 0) {
            sh.ncand = 0u;
            sh.overflow = 0u;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float x = elem(xv[q >> 2], q & 3);
            const float t = fmaf(x, c, -R);
            const int b = (x > -INFINITY)
                              ? (int)fminf(fmaxf(-t * kSampleRes, 0.0f), (float)(kSampleBins - 1))
                              : kSampleBins + l;  // -inf (outside the row or masked): dummy bin
            atomicAdd(&sh.scnt[b], 1u);
        }
        lds_barrier();
    }

    // ====================================================================
    // Dense route
    // ---- T2: value window bracketing the cutoff, from the sample (wave 0)
    if (topp && w == 0) {
        // lane l owns bins [8l, 8l + 8); bin 0 = top of the row
        uint32_t cnt = 0;
        float msf = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < kBinsPerLane / 4; ++i4) {
            const u4v sb = *reinterpret_cast<const u4v*>(&sh.scnt[kBinsPerLane * l + 4 * i4]);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t n = elemu(sb, q);
                cnt += n;
                msf += (float)n * bin_mass(kBinsPerLane * l + 4 * i4 + q);
            }
        }
        const uint32_t cnt_incl = wscan_u32(cnt);
        const double ms_incl = wscan_f64((double)msf);
        const uint32_t n_s = (uint32_t)__builtin_amdgcn_readlane((int)cnt_incl, 63);
        const double S_s = bcast_f64(ms_incl, 63);
        // estimated boundary: the sample rank at which the mass left below
        // (sample mass scaled to the row) drops to (1 - p) * Z
        const double F = (double)V / (double)max(n_s, 1u);
        const double removed = (1.0 - (double)p) * ZR;
        int n_above = 0;
        if (F * S_s > removed) {
            const uint64_t bal = __ballot(F * (S_s - ms_incl) <= removed);
            const int L0 = bal ? (__ffsll((long long)bal) - 1) : 63;
            int na_l = -1;
            if (l == L0) {
                double mprev = ms_incl - (double)msf;
                int na = (int)(cnt_incl - cnt);
                bool done = false;
                #pragma unroll 1
                for (int i = 0; i < kBinsPerLane; ++i) {
                    if (!done) {
                        const uint32_t n = sh.scnt[kBinsPerLane * l + i];
                        mprev += (double)((float)n * bin_mass(kBinsPerLane * l + i));
                        na += (int)n;
                        done = F * (S_s - mprev) <= removed;
                    }
                }
                na_l = na;
            }
            n_above = __shfl(na_l, L0);
        }
        const int n_below = (int)n_s - n_above;
        const int W = (int)(6.0 * sqrt((double)min(n_above, n_below))) + 10;
        const int top_rank = n_above - W;  // sample ranks (from the top) bracketing the cutoff
        const int bot_rank = n_above + W;
        const int cexcl = (int)(cnt_incl - cnt);
        // the bin holding a given sample rank (read back from LDS by its owner lane)
        int b_top = -1, b_bot = kSampleBins;
#define NIS_BIN_OF_RANK(rank, out)                                   \
    {                                                                \
        const uint64_t bal = __ballot((int)cnt_incl >= (rank));      \
        const int L = __ffsll((long long)bal) - 1;                   \
        int b = -1;                                                  \
        if (l == L) {                                                \
            int acc = cexcl;                                         \
            for (int i = 0; i < kBinsPerLane; ++i) {                           \
                acc += (int)sh.scnt[kBinsPerLane * l + i];                     \
                if (b < 0 && acc >= (rank)) b = kBinsPerLane * l + i;          \
            }                                                        \
        }                                                            \
        (out) = __shfl(b, L);                                        \
    }
        if (top_rank > 0) NIS_BIN_OF_RANK(top_rank, b_top)
        if (bot_rank < (int)n_s) NIS_BIN_OF_RANK(bot_rank, b_bot)
#undef NIS_BIN_OF_RANK
        {
            // never leave the window open below: stop at the lowest sample
            // bin (a cutoff below it is caught by the bottom check)
            const uint64_t nzb = __ballot(cnt != 0);
            if (nzb) {
                const int L = 63 - __clzll((long long)nzb);
                int lb = -1;
                if (l == L) {
                    #pragma unroll 1
                    for (int i = 0; i < kBinsPerLane; ++i)
                        if (sh.scnt[kBinsPerLane * l + i] != 0) lb = kBinsPerLane * l + i;
                }
                lb = __shfl(lb, L);
                if (b_bot > lb) b_bot = lb;
            }
        }
        if (l == 0) {
            // bin b holds t in (-(b+1)/64, -b/64]; the elements above bin
            // b_top are kept for sure, the window spans bins b_top..b_bot
            sh.bf[0] = (b_top < 0) ? INFINITY : ((float)(-b_top) / kSampleRes + R) / c;
            sh.bf[1] = (b_bot >= kSampleBins) ? -INFINITY
                                              : ((float)(-(b_bot + 1)) / kSampleRes + R) / c;
        }
    }
    if (topp) lds_barrier();
    NIS_TS(10);
    // without top-p every finite element is kept and the window is empty
    const float x_hi = topp ? sh.bf[0] : -INFINITY;
    const float x_lo = topp ? sh.bf[1] : INFINITY;

    // ---- P1: per-chunk kept mass above the window, window elements listed
    double lane_kept = 0.0;  // kept mass of this lane (R-units)
    int nsure = 0;           // kept elements of this lane above the window
    int lpos = 0;            // window elements of this lane
#pragma unroll
    for (int k = 0; k < kNch; ++k) {
        float cs = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float x = elem(xv[k], q);
            const bool sure = x > x_hi;
            cs += sure ? mass_of(x, c, R) : 0.0f;
            nsure += sure ? 1 : 0;
            if (!sure && x >= x_lo) {
                if (lpos < kLaneCap) {
                    sh.d.lx[lpos][tid] = x;
                    sh.d.lp[lpos][tid] = (uint8_t)(4 * k + q);
                }
                ++lpos;
            }
        }
        sh.d.cell[w][k][l] = cs;
        lane_kept += (double)cs;
    }
    // the window's fine histogram (count, mass, largest and smallest key)
    if (topp && lpos <= kLaneCap) {
        const float x_top = fminf(x_hi, M);
        const float inv_wd = (x_top > x_lo) ? (float)kFineBins / (x_top - x_lo) : 0.0f;
        const double sfix = rho * kFix;
        #pragma unroll 1
        for (int i = 0; i < lpos; ++i) {
            const float x = sh.d.lx[i][tid];
            const int fb = fine_bucket(x, x_lo, inv_wd);
            const uint32_t key = key32(x);
            atomicAdd(&sh.fcnt[fb], 1u);
            atomicAdd(&sh.fmass[fb], (unsigned long long)((double)mass_of(x, c, R) * sfix));
            atomicMax(&sh.fkmax[fb], key);
            atomicMin(&sh.fkmin[fb], key);
        }
    }
    if (lpos > kLaneCap) sh.overflow = 1u;
    {
        const double g = wsum_f64(lane_kept);
        NIS_PUT(l == 0, sh.db[w], g);
    }
    lds_barrier();
    NIS_TS(11);
    if (sh.overflow) return reject != NIS_REJECT_NONE ? reject : NIS_REJECT_CAPACITY;
    const int nl = lpos;  // <= kLaneCap here

    float xf_lo = INFINITY, xf_hi = -INFINITY;  // value range of the cutoff bucket
    double g_above_f = 0.0;
    uint32_t n_final = 0;
    if (topp) {
        double GhiR = sh.db[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) GhiR += sh.db[i];

        // ---- T4: the fine bucket holding the cutoff (wave 0) -------------
        if (w == 0) {
            // lane l owns buckets 1008-16l .. 1023-16l; index i = 15 is the
            // top one (descending value runs i = 15 .. 0, then the next lane)
            const int b0 = kFineBins - 16 - 16 * l;
            uint32_t cnt[16], kmx[16];
            unsigned long long fm[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const u4v cv = *reinterpret_cast<const u4v*>(&sh.fcnt[b0 + i]);
                const u4v kv = *reinterpret_cast<const u4v*>(&sh.fkmax[b0 + i]);
                cnt[i] = cv.x; cnt[i + 1] = cv.y; cnt[i + 2] = cv.z; cnt[i + 3] = cv.w;
                kmx[i] = kv.x; kmx[i + 1] = kv.y; kmx[i + 2] = kv.z; kmx[i + 3] = kv.w;
            }
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const u4v mv = *reinterpret_cast<const u4v*>(&sh.fmass[b0 + i]);
                fm[i] = ((unsigned long long)mv.y << 32) | mv.x;
                fm[i + 1] = ((unsigned long long)mv.w << 32) | mv.z;
            }
            unsigned long long mlf = 0;  // the lane's mass in fixed point (exact sum)
#pragma unroll
            for (int i = 0; i < 16; ++i) mlf += fm[i];
            const double mlane = (double)mlf / kFix;
            const double incl = wscan_f64(mlane);
            const double Ghi = GhiR * rho;
            // mass above each bucket, walking down the lane's buckets; a
            // bucket qualifies if its largest element is kept (sampler.rs:150)
            double G = Ghi + (incl - mlane);
            int lowq = kFineBins;       // lowest qualifying bucket of this lane
            double gq = 0.0;            // mass above it
            int lastne = kFineBins;     // lowest non-empty bucket of this lane
            bool stop = false;
#pragma unroll
            for (int i = 15; i >= 0; --i) {
                const bool ne = cnt[i] != 0;
                const double ef = (double)mass_of(unkey32(kmx[i]), c, R) * rho;
                const bool q = ne & !stop & (G - ef <= pZ);
                stop = stop | (ne & !q);
                lowq = q ? (b0 + i) : lowq;
                gq = q ? G : gq;
                lastne = ne ? (b0 + i) : lastne;
                G += (double)fm[i] / kFix;
            }
            // qualifying buckets form a prefix from the top: the cutoff
            // bucket is the lowest of them (DPP minima of bucket indices;
            // exact in float)
            const float lowf = -wmax_f32(-(float)lowq);
            const int best = (int)lowf;
            const float nef = -wmax_f32(-(float)lastne);
            const int lowest = (int)nef;
            const double Gtot = bcast_f64(incl, 63) + Ghi;
            const uint64_t own = __ballot(lowq == best);
            const int owner = own ? (__ffsll((long long)own) - 1) : 0;
            const double gs = bcast_f64(gq, owner);
            int ok = 1;
            // every element above the window must be kept
            if (x_hi < INFINITY && !(Ghi - (double)mass_of(x_hi, c, R) * rho <= pZ)) ok = 0;
            if (best >= kFineBins) ok = 0;
            // cutoff in the lowest bucket: the first element below the
            // window must be removed
            if (ok && best == lowest && !(Gtot - (double)mass_of(x_lo, c, R) * rho > pZ)) ok = 0;
            NIS_PUT(l == 0, sh.bi[0], ok);
            NIS_PUT(l == 0, sh.bi[1], ok ? best : 0);
            NIS_PUT(l == 0, sh.bd[0], gs);
        }
        lds_barrier();
        NIS_TS(12);
        if (!sh.bi[0]) return NIS_REJECT_WINDOW;
        const int fstar = sh.bi[1];
        n_final = sh.fcnt[fstar];
        if (n_final > (uint32_t)kMaxFinal) return NIS_REJECT_CAPACITY;
        xf_hi = unkey32(sh.fkmax[fstar]);
        xf_lo = unkey32(sh.fkmin[fstar]);
        g_above_f = sh.bd[0];
        // flag list entries above the bucket as kept, gather the bucket's members
        #pragma unroll 1
        for (int i = 0; i < nl; ++i) {
            const float x = sh.d.lx[i][tid];
            if (x > xf_hi) {
                sh.d.lp[i][tid] |= kKeptBit;
            } else if (x >= xf_lo) {
                const uint32_t s = atomicAdd(&sh.ncand, 1u);
                if (s < (uint32_t)kMaxFinal) {
                    const int pos = sh.d.lp[i][tid];
                    sh.d.cj[s] = (uint32_t)(4 * (slot0 + 64 * (pos >> 2)) + (pos & 3) - mis);
                    sh.d.cx[s] = x;
                    sh.d.cloc[s] = (uint32_t)(tid * kLaneCap + i);
                }
            }
        }
        lds_barrier();
        if (sh.ncand != n_final) return NIS_REJECT_BUCKET;  // bucket membership must match the histogram

        // ---- T6: exact rule on the cutoff bucket (wave 0) -------------------
        if (w == 0) {
            const int n = (int)n_final;
            const bool valid = l < n;
            const int lc = min(l, kMaxFinal - 1);
            const float cxv = sh.d.cx[lc];
            const uint32_t cjv = sh.d.cj[lc];
            const float xm = valid ? cxv : -INFINITY;
            const uint32_t km = key32(xm);
            const uint32_t im = valid ? cjv : 0u;
            const double em = valid ? (double)mass_of(xm, c, R) * rho : 0.0;
            double pre = 0.0;  // mass of the members ahead in the stable descending order
            #pragma unroll 1
            for (int j = 0; j < n; ++j) {
                const uint32_t kj = bcast_u32(km, j), ij = bcast_u32(im, j);
                const double ej = bcast_f64(em, j);
                pre += ((kj > km) | ((kj == km) & (ij < im))) ? ej : 0.0;
            }
            // sampler.rs:150: removed iff cum_excl - q > p; kept otherwise
            const bool kept = valid & (g_above_f + pre - em <= pZ);
            if (kept) {
                const uint32_t loc = sh.d.cloc[l];
                sh.d.lp[loc % kLaneCap][loc / kLaneCap] |= kKeptBit;
            }
        }
        lds_barrier();
    }
    NIS_TS(13);

    // ---- T7: inverse-CDF walk in index order --------------------------------
    // kept list entries join their lane's cells (the owner updates its own cells)
    int nkept = nsure;
    #pragma unroll 1
    for (int i = 0; i < nl; ++i) {
        const int pos = sh.d.lp[i][tid];
        if (pos & kKeptBit) {
            const int k = (pos & 0x7F) >> 2;
            const float e = mass_of(sh.d.lx[i][tid], c, R);
            sh.d.cell[w][k][l] += e;
            lane_kept += (double)e;
            ++nkept;
        }
    }
    {
        const double wt = wsum_f64(lane_kept);
        const int wk = (int)wsum_u32((uint32_t)nkept);
        if (l == 0) {
            sh.wtot[w] = wt;
            sh.ia[w] = wk;
        }
    }
    lds_barrier();
    // per-wave totals (lanes 0..7), their prefix and the wave holding the
    // crossing: the first whose running total reaches r (and has mass);
    // rounding: the last wave with mass
    const double u = sh.bd[1];
    double zk, r, wbase;
    int wsel;
    {
        const int li = min(l, kWaves - 1);
        const double Tw = (l < kWaves) ? sh.wtot[li] : 0.0;
        const double Twi = wscan_f64(Tw);
        zk = bcast_f64(Twi, 63);
        r = u * zk;
        const uint64_t hw = __ballot((l < kWaves) & (Tw > 0.0) & (Twi >= r));
        const uint64_t nzw = __ballot((l < kWaves) & (Tw > 0.0));
        wsel = hw ? (__ffsll((long long)hw) - 1) : (nzw ? (63 - __clzll((long long)nzw)) : 0);
        wbase = bcast_f64(Twi - Tw, wsel);
    }
    wsel = __builtin_amdgcn_readfirstlane(wsel);
    if (w == wsel) {  // static register indices only (a dynamic one would demote xv to scratch)
#pragma unroll
        for (int k = 0; k < kNch; ++k) sh.d.stx[k][l] = xv[k];
    }
    // chunk totals of the chosen wave (wave w handles chunks w, w+8, ...)
    #pragma unroll 1
    for (int kk = w; kk < kNch; kk += kWaves) {
        const double cv = wsum_f64((double)sh.d.cell[wsel][kk][l]);
        NIS_PUT(l == 0, sh.ctot[kk], cv);
    }
    lds_barrier();
    // the chunk holding the crossing (lanes 0..kNch-1), as for the waves
    int ksel;
    double kbase;
    {
        const int lk = min(l, kNch - 1);
        const double Ck = (l < kNch) ? sh.ctot[lk] : 0.0;
        const double Cki = wscan_f64(Ck);
        const uint64_t hk = __ballot((l < kNch) & (Ck > 0.0) & (wbase + Cki >= r));
        const uint64_t nzk = __ballot((l < kNch) & (Ck > 0.0));
        ksel = hk ? (__ffsll((long long)hk) - 1) : (nzk ? (63 - __clzll((long long)nzk)) : 0);
        kbase = wbase + bcast_f64(Cki - Ck, ksel);
    }
    ksel = __builtin_amdgcn_readfirstlane(ksel);
    if (w == wsel) {
        // lane prefix inside the chosen chunk; the owning lane finishes the walk
        const double cvl = (double)sh.d.cell[wsel][ksel][l];
        const double incl = wscan_f64(cvl);
        const uint64_t hit = __ballot(kbase + incl >= r && cvl > 0.0);
        const uint64_t nz = __ballot(cvl > 0.0);
        const int lsel = hit ? (__ffsll((long long)hit) - 1) : (63 - __clzll((long long)nz));
        if (l == lsel) {
            // this lane's kept flags for the chunk's 4 elements
            uint32_t wkept = 0;
            #pragma unroll 1
            for (int i = 0; i < nl; ++i) {
                const int pos = sh.d.lp[i][tid];
                if ((pos & kKeptBit) && ((pos & 0x7F) >> 2) == ksel) wkept |= 1u << (pos & 3);
            }
            const f4v xs = sh.d.stx[ksel][l];
            double run = kbase + incl - cvl;
            int tok = -1, last = -1;
            float xt = 0.0f, xlast = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float x = elem(xs, q);
                if (x > x_hi || ((wkept >> q) & 1u)) {
                    run += (double)mass_of(x, c, R);
                    const int j = 4 * (slot0 + 64 * ksel) + q - mis;
                    if (tok < 0) {
                        last = j;
                        xlast = x;
                        if (run >= r) {
                            tok = j;
                            xt = x;
                        }
                    }
                }
            }
            bool tkept = true;
            if (tok < 0) {  // rounding: the crossing is this lane's last kept token
                tok = last;
                xt = xlast;
            }
            if (u == 0.0) {  // r == 0 stops the reference's walk at index 0 (sampler.rs:210-213)
                tok = 0;
                tkept = false;
            }
            int kept_total = 0;
            #pragma unroll 1
            for (int i = 0; i < kWaves; ++i) kept_total += sh.ia[i];
            const double zkM = zk * rho;
            const double prob = tkept ? (double)mass_of(xt, c, R) / zk : 0.0;
            // `reject`: why the sparse route declined this row (0 without top-p)
            write_row_result(a, row, (uint32_t)tok, NIS_PATH_DRAW, (double)M / temp, zkM,
                             topp ? ZR * rho : 0.0, u, prob, (uint64_t)kept_total, 1, reject);
        }
    }
    if (tid == 0) {
        uint64_t* sp = a.rng + 4 * (int64_t)row;
        sp[0] = sh.rng[0];
        sp[1] = sh.rng[1];
        sp[2] = sh.rng[2];
        sp[3] = sh.rng[3];
    }
    NIS_TS(14);
    return NIS_REJECT_NONE;
#undef NIS_FIX
#undef NIS_INDEX
}

}  // namespace nis
