// lm_head.h — the LM-head producer: logits[b][v] = dot(hidden[b], W[v]) for
// B last-hidden rows, on the matrix cores.
//
// Reference: Model::logits_last (src/model.rs:317-325) calls Mat::gemv_into
// (src/model.rs:65-86) on the LM head or the tied embedding; a dense row is
// simd::dot_f32 (src/simd.rs:22), a quantized one QuantMatrix::dot_rows_into
// (src/quant.rs:121-161): int8 biased bytes or int4 biased nibbles (low nibble
// first over the global index row*H + k), one f32 scale per row applied to the
// row's dot product, or one per group of input channels applied to each
// group's partial dot product.
//
// Layout and tiling (gfx950):
//   - v_mfma_f32_16x16x4_f32, A = 16 hidden rows (b), B = 16 weight rows (v):
//     lane l holds row l%16 at reduction index l/16 of each operand, and
//     D[b = 4*(l/16) + r][v = l%16] in accumulator r.  The reduction index is
//     permuted so that a lane's four successive MFMAs use four consecutive h:
//     each operand is one 16-byte load per lane per four MFMAs.
//   - A wave owns 64 vocab rows x 16*NB hidden rows (4 x NB accumulator tiles)
//     and walks h in chunks of 16 (f32) or 32 (packed codes: two runs of 4
//     per lane), with the next chunk's loads issued before the current
//     chunk's MFMAs.
//   - Quantized codes stay packed until the MFMAs of their chunk: int8 runs
//     are one u32, int4 runs one u16; (code - bias) is exact in f32.  A
//     per-row scale multiplies the finished dot product, as in the
//     reference; a group scale multiplies each weight (same real value, one
//     more rounding per term, inside the f32 error bound of the sum).
//   - Stores: accumulator r of a tile is 4 hidden rows x 16 consecutive
//     vocab entries, 64 contiguous bytes per row.
// The split form (KS > 1, at 4 hidden tiles per wave) passes partial sums
// through LDS behind one barrier; otherwise no LDS and no barriers.  Waves
// outside the problem do no work (and, in the split form, still reach the
// barrier); every load index is clamped into the operands and every store
// is masked.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "device_common.h"

namespace nis {

typedef float lh_f4 __attribute__((ext_vector_type(4)));


enum { kLhF32 = 0, kLhInt4 = 4, kLhInt8 = 8 };

struct LmHeadArgs {
    const float* x;        // hidden [B][ldx]
    int64_t ldx;
    int32_t B;
    int32_t H;
    const void* w;         // weights, row v of H entries (f32, u8 or packed u4)
    const float* scales;   // [V][groups] (quantized only)
    int32_t group;         // group length (H when one scale per row)
    int32_t groups;        // H / group
    uint32_t gmagic;       // ceil(2^32 / group); 0 for group 1 (2^32 does not fit)
    int32_t wv;            // waves of a workgroup along v (wv * wb waves)
    int32_t wb;            // waves of a workgroup along b
    int32_t hs;            // KS > 1: length of each part of h but the last (whole chunks)
    int32_t gx;            // KS > 1: workgroups along b
    int64_t V;
    float* out;            // logits [B][ld] (greedy form: may be null)
    int64_t ld;
    unsigned long long* part;  // greedy form: one key per workgroup (lh_greedy_key)
};

// Greedy order of one logit (sampler.rs:172-181: the first index of the
// maximum; a NaN at index 0 stops every comparison, so index 0 wins; any
// other NaN never wins): larger keys win, and on equal values the lower index
// (its complement sits in the low half).
__device__ __forceinline__ unsigned long long lh_greedy_key(float x, int64_t v) {
    const uint32_t lo = 0xFFFFFFFFu - (uint32_t)v;
    if (x != x) return v == 0 ? ~0ull : (((unsigned long long)key32(-INFINITY) << 32) | lo);
    return ((unsigned long long)key32(x) << 32) | lo;
}
__device__ __forceinline__ unsigned long long lh_wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long t = (unsigned long long)__shfl_xor((long long)k, o);
        k = t > k ? t : k;
    }
    return k;
}

// floor(h / group) for 0 <= h < 2^31: the product with ceil(2^32/group) is
// exact or one too high.  Group 1 (magic 0) is h itself.
__device__ __forceinline__ int lh_group_of(const LmHeadArgs& a, int h) {
    if (a.gmagic == 0u) return h;
    int q = (int)__umulhi((uint32_t)h, a.gmagic);
    return q * a.group > h ? q - 1 : q;
}

__device__ __forceinline__ float lh_code(const LmHeadArgs& a, int64_t idx, int fmt) {
    const uint8_t* q = (const uint8_t*)a.w;
    if (fmt == kLhInt8) return (float)((int)q[idx] - 128);
    uint8_t byte = q[idx >> 1];
    return (float)((int)((idx & 1) ? (byte >> 4) : (byte & 15)) - 8);
}

// Hidden run h..h+3 of row `row` (zero past H).
template <bool VEC>
__device__ __forceinline__ lh_f4 lh_load_x(const LmHeadArgs& a, int64_t row, int h) {
    lh_f4 r = {0.f, 0.f, 0.f, 0.f};
    const float* p = a.x + row * a.ldx;
    if (VEC) {
        if (h < a.H) r = *(const lh_f4*)(p + h);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (h + e < a.H) r[e] = p[h + e];
    }
    return r;
}

// A weight run in flight: the raw 16 bytes / u32 / u16 and, for group scales,
// the run's scale (a run never straddles a group when VEC holds).
struct LhRun {
    lh_f4 f;
    uint32_t c;
    float s;
};

template <int FMT, bool VEC, bool GROUPED>
__device__ __forceinline__ LhRun lh_load_w(const LmHeadArgs& a, int64_t v, int h) {
    LhRun r;
    r.f = lh_f4{0.f, 0.f, 0.f, 0.f};
    r.c = FMT == kLhInt8 ? 0x80808080u : 0x8888u;  // codes of 0.0 past H
    r.s = 0.f;
    const int64_t base = v * (int64_t)a.H;
    if (VEC) {
        if (h < a.H) {
            if (FMT == kLhF32) {
                r.f = *(const lh_f4*)((const float*)a.w + base + h);
            } else if (FMT == kLhInt8) {
                r.c = *(const uint32_t*)((const uint8_t*)a.w + base + h);
            } else {
                r.c = *(const uint16_t*)((const uint8_t*)a.w + ((base + h) >> 1));
            }
            if (GROUPED) r.s = a.scales[v * a.groups + lh_group_of(a, h)];
        }
    } else {
        // any H, any group length: dequantized here, element by element
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (h + e >= a.H) continue;
            if (FMT == kLhF32) {
                r.f[e] = ((const float*)a.w)[base + h + e];
            } else {
                float c = lh_code(a, base + h + e, FMT);
                r.f[e] = GROUPED ? c * a.scales[v * a.groups + lh_group_of(a, h + e)] : c;
            }
        }
    }
    return r;
}

template <int FMT, bool VEC, bool GROUPED>
__device__ __forceinline__ lh_f4 lh_values(const LhRun& r) {
    if (FMT == kLhF32 || !VEC) return r.f;
    lh_f4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float c = FMT == kLhInt8 ? (float)((int)((r.c >> (8 * e)) & 255u) - 128)
                                 : (float)((int)((r.c >> (4 * e)) & 15u) - 8);
        w[e] = GROUPED ? c * r.s : c;
    }
    return w;
}

// KS > 1: KS waves of a workgroup share each tile, each summing one part of
// h (a.hs long, a whole number of chunks; the last part takes the rest);
// the accumulators of parts 1..KS-1 go through LDS and the part-0 wave adds
// them in that fixed order as it stores.  Finer work items spread
// the launch evenly over the SIMDs: at B = 256, V = 50257, 3144 whole tiles
// fill 3 waves per SIMD and leave 72 over, which run on after the rest.
template <int FMT, bool VEC, bool GROUPED, int NB, int KS>
__global__ __launch_bounds__(256) void lm_head_kernel(LmHeadArgs a) {
    // runs of 4 h per lane per chunk: one for f32 (100 VGPRs, 3 waves per
    // SIMD: 260 us at B = 256 against 281 with two), two for packed codes
    // (their loads are narrower; one run was 4 % slower for int4)
    constexpr int kLhRuns = FMT == kLhF32 ? 1 : 2;
    const int lane = threadIdx.x & 63;
    const int wave = (threadIdx.x >> 6) % (a.wv * a.wb);  // the tile's wave
    const int ks = (threadIdx.x >> 6) / (a.wv * a.wb);    // KS > 1: its part of h
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    // KS > 1: a 1-D grid, mapped so that the a.gx workgroups of one vocab
    // tile get ids 8 apart: the dispatcher deals ids round-robin over the 8
    // XCDs, so they share one L2 and the tile's weights are fetched once
    int64_t bx = blockIdx.x, by = blockIdx.y;
    if constexpr (KS > 1) {
        const int64_t id = blockIdx.x, k = id >> 3;
        bx = k % a.gx;
        by = 8 * (k / a.gx) + (id & 7);
    }
    const int64_t b0 = (bx * a.wb + wave / a.wv) * (16 * NB);
    const int64_t v0 = (by * a.wv + wave % a.wv) * 64;
    const bool live = b0 < a.B && v0 < a.V;
    if (KS == 1 && !live) return;
    const int hbeg = KS == 1 ? 0 : ks * a.hs;
    const int hend = (KS == 1 || ks == KS - 1) ? a.H : min(a.H, (ks + 1) * a.hs);

    int64_t vrow[4], brow[NB];
#pragma unroll
    for (int j = 0; j < 4; ++j) vrow[j] = min(v0 + 16 * j + r16, a.V - 1);
#pragma unroll
    for (int i = 0; i < NB; ++i) brow[i] = min(b0 + 16 * i + r16, (int64_t)a.B - 1);

    lh_f4 acc[NB][4];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = lh_f4{0.f, 0.f, 0.f, 0.f};

    // KS = 1: the next chunk's loads go out before this chunk's MFMAs.  KS > 1
    // loads each chunk as it starts it (the prefetch's registers would take
    // the third wave per SIMD; the other waves cover the loads' latency).
    constexpr bool kPF = KS == 1;
    lh_f4 xc[NB][kLhRuns];
    LhRun wc[4][kLhRuns];
#pragma unroll
    for (int s = 0; s < kLhRuns; ++s) {
#pragma unroll
        for (int i = 0; i < NB; ++i) xc[i][s] = lh_load_x<VEC>(a, brow[i], hbeg + 16 * s + 4 * kq);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            wc[j][s] = lh_load_w<FMT, VEC, GROUPED>(a, vrow[j], hbeg + 16 * s + 4 * kq);
    }
    for (int h0 = hbeg; live && h0 < hend; h0 += 16 * kLhRuns) {
        lh_f4 xn[NB][kLhRuns];
        LhRun wn[4][kLhRuns];
        const int hn = h0 + 16 * kLhRuns;  // past H the loads return zeros / zero codes
        if constexpr (kPF) {
#pragma unroll
            for (int s = 0; s < kLhRuns; ++s) {
#pragma unroll
                for (int i = 0; i < NB; ++i) xn[i][s] = lh_load_x<VEC>(a, brow[i], hn + 16 * s + 4 * kq);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    wn[j][s] = lh_load_w<FMT, VEC, GROUPED>(a, vrow[j], hn + 16 * s + 4 * kq);
            }
        }
#pragma unroll
        for (int s = 0; s < kLhRuns; ++s) {
            lh_f4 wv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) wv[j] = lh_values<FMT, VEC, GROUPED>(wc[j][s]);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int i = 0; i < NB; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[i][s][c], wv[j][c],
                                                                         acc[i][j], 0, 0, 0);
        }
        // (without prefetch the next chunk is loaded only while one is left in
        // this part's range: the last iteration issues no loads past hend)
        if (kPF || hn < hend) {
#pragma unroll
            for (int s = 0; s < kLhRuns; ++s) {
#pragma unroll
                for (int i = 0; i < NB; ++i)
                    xc[i][s] = kPF ? xn[i][s] : lh_load_x<VEC>(a, brow[i], hn + 16 * s + 4 * kq);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    wc[j][s] = kPF ? wn[j][s] : lh_load_w<FMT, VEC, GROUPED>(a, vrow[j], hn + 16 * s + 4 * kq);
            }
        }
    }

    // [part - 1][tile wave][accumulator][lane]: the sums of parts 1..KS-1
    // (KS > 1: a workgroup holds 4 / KS tile waves)
    constexpr int kTw = KS > 1 ? 4 / KS : 1;
    __shared__ float part[KS > 1 ? KS - 1 : 1][kTw][KS > 1 ? NB * 16 : 1][64];
    if constexpr (KS > 1) {
        if (ks > 0) {
#pragma unroll
            for (int i = 0; i < NB; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) part[ks - 1][wave][16 * i + 4 * j + r][lane] = acc[i][j][r];
        }
        __syncthreads();
        if (ks > 0 || !live) return;
    }
    // (KS > 1: the other parts are added, in order, as each value is stored)
    const float* const pw = KS > 1 ? &part[0][wave][0][lane] : nullptr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t v = v0 + 16 * j + r16;
        if (v >= a.V) continue;
        const float sc = (FMT != kLhF32 && !GROUPED) ? a.scales[v] : 1.0f;
#pragma unroll
        for (int i = 0; i < NB; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t b = b0 + 16 * i + 4 * kq + r;
                if (b < a.B) {
                    float y = acc[i][j][r];
#pragma unroll
                    for (int p = 1; p < KS; ++p)  // ((part 0 + part 1) + part 2) + ...
                        y += pw[64 * ((p - 1) * kTw * NB * 16 + 16 * i + 4 * j + r)];
                    if (FMT != kLhF32 && !GROUPED) y *= sc;  // dot * scale (quant.rs:128)
                    a.out[b * a.ld + v] = y;
                }
            }
    }
}

// One hidden row (B = 1, the reference's own decode shape): matrix-core tiles
// would pad it to 16 rows, so this is a VALU GEMV streaming the head once.
// Each lane takes runs of R codes (16 bytes: 4 f32 or 16 int8; 8 bytes: 16
// int4) at fixed h positions j*R, j = li + k*L (k < KM), of one weight row;
// L (16 or 64) lanes share a row, 64/L rows per wave step, ITER steps per
// wave.  The lane's hidden values for those positions stay in registers
// across the steps, with their sum per run; the runs of D steps are in
// flight while a step is summed; the L partial sums of a row meet in a DPP
// scan (fixed order, deterministic).
//
// A quantized code is converted as the unsigned byte it is stored in (one
// v_cvt_f32_ubyte per code: int8 bytes as they are, int4 nibbles spread one
// per byte first), and the zero point (128, 8) comes off once per run:
// sum (q - z) x = sum q x - z sum x.  The issue slots per code (one convert,
// one fma) bound these kernels, not their bytes.

template <int FMT>
struct LhRowCfg {
    static constexpr int R = FMT == kLhF32 ? 4 : 16;                         // h per run
    static constexpr int RB = FMT == kLhInt4 ? 8 : 16;                      // bytes per run
    // measured at H = 768, V = 50257 (wave steps, steps in flight): int8
    // (4, 2) against (2, 2) (4, 4) (8, 4) (8, 8); int4 (4, 4) against (8, 8)
    // (8, 4) (16, 8); f32 (4, 4)
    static constexpr int ITER = 4;                                          // wave steps
    static constexpr int D = FMT == kLhInt8 ? 2 : ITER;                     // steps in flight
};
template <int FMT> struct LhRunT { typedef uint4 T; };
template <> struct LhRunT<kLhInt4> { typedef uint2 T; };

// sum over the run of code * x, the zero point taken off with the run's sum of x
template <int FMT>
__device__ __forceinline__ float lh_run_dot(const typename LhRunT<FMT>::T& raw, const float* xr, float sx) {
    constexpr int R = LhRowCfg<FMT>::R;
    float part = 0.f;
    if constexpr (FMT == kLhF32) {
        const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < R; ++e) part = fmaf(__uint_as_float(wd[e]), xr[e], part);
        return part;
    } else if constexpr (FMT == kLhInt8) {
        const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < R; ++e) part = fmaf((float)((wd[e >> 2] >> (8 * (e & 3))) & 255u), xr[e], part);
        return fmaf(-128.0f, sx, part);
    } else {
        // code e: word e/8, byte (e%8)/2, the low nibble for even e
        const uint32_t wd[2] = {raw.x, raw.y};
#pragma unroll
        for (int wi = 0; wi < 2; ++wi) {
            uint32_t lo = wd[wi] & 0x0F0F0F0Fu, hi = (wd[wi] >> 4) & 0x0F0F0F0Fu;
            asm("" : "+v"(lo), "+v"(hi));  // (the masks hidden: byte conversions, not bit extracts)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                part = fmaf((float)((lo >> (8 * b)) & 255u), xr[8 * wi + 2 * b], part);
                part = fmaf((float)((hi >> (8 * b)) & 255u), xr[8 * wi + 2 * b + 1], part);
            }
        }
        return fmaf(-8.0f, sx, part);
    }
}

// GREEDY: greedy decoding fused into the epilogue.  Each lane holding a
// finished row keeps the best greedy key of its rows; the workgroup's best
// goes to a.part[blockIdx.x], and lm_head_greedy_final_kernel reduces those.
// (The last workgroup to finish reducing them instead needs a release fence
// per workgroup, which writes the L2 back each time: far slower.)
template <int FMT, bool GROUPED, bool GREEDY, int KM>
__global__ __launch_bounds__(256) void lm_head_row_kernel(LmHeadArgs a, int log2L, int runs) {
    constexpr int R = LhRowCfg<FMT>::R;
    constexpr int RB = LhRowCfg<FMT>::RB;
    typedef typename LhRunT<FMT>::T RunT;
    const int lane = threadIdx.x & 63;
    const int L = 1 << log2L;
    const int li = lane & (L - 1);
    const int P = 64 >> log2L;
    constexpr int ITER = LhRowCfg<FMT>::ITER;
    const int64_t wave_row0 = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * P * ITER;
    __shared__ unsigned long long gk[GREEDY ? 4 : 1];  // greedy: each wave's best key
    if (wave_row0 >= a.V) {  // wave-uniform
        if (GREEDY) {
            if (lane == 0) gk[threadIdx.x >> 6] = 0ull;
            __syncthreads();
            if (threadIdx.x == 0) a.part[blockIdx.x] = max(max(gk[0], gk[1]), max(gk[2], gk[3]));
        }
        return;
    }
    unsigned long long best = 0ull;  // greedy: this lane's best key
    const int gl = lane >> log2L;
    const int64_t row_bytes = FMT == kLhF32 ? (int64_t)a.H * 4 : (FMT == kLhInt8 ? (int64_t)a.H : (int64_t)a.H / 2);

    constexpr int D = LhRowCfg<FMT>::D;
    RunT ring[D][KM];
    auto load_step = [&](int it, RunT* dst) {
        const int64_t vl = min(wave_row0 + it * P + gl, a.V - 1);
        const uint8_t* wrow = (const uint8_t*)a.w + vl * row_bytes;
#pragma unroll
        for (int k = 0; k < KM; ++k) {
            // (every load made, from an address clamped into the row, and
            // zeroed after: no branch around a load)
            const int j = li + k * L;
            const RunT v = *(const RunT*)(wrow + (int64_t)min(j, runs - 1) * RB);
            RunT z{};
            dst[k] = j < runs ? v : z;
        }
    };
#pragma unroll
    for (int it = 0; it < D; ++it) load_step(it, ring[it]);
    float xr[KM][R];
    float sx[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        const int j = li + k * L;
        sx[k] = 0.f;
#pragma unroll
        for (int q = 0; q < R / 4; ++q) {
            const lh_f4 xl = *(const lh_f4*)(a.x + (int64_t)min(j, runs - 1) * R + 4 * q);
            const lh_f4 xv = j < runs ? xl : lh_f4{0.f, 0.f, 0.f, 0.f};
            xr[k][4 * q] = xv[0];
            xr[k][4 * q + 1] = xv[1];
            xr[k][4 * q + 2] = xv[2];
            xr[k][4 * q + 3] = xv[3];
            sx[k] += (xv[0] + xv[1]) + (xv[2] + xv[3]);
        }
    }
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        const int64_t v = wave_row0 + it * P + gl;
        const int64_t vl = min(v, a.V - 1);
        RunT cur[KM];
#pragma unroll
        for (int k = 0; k < KM; ++k) cur[k] = ring[it % D][k];
        if (it + D < ITER) load_step(it + D, ring[it % D]);
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < KM; ++k) {
            const int j = li + k * L;
            if (j < runs) {
                const float part = lh_run_dot<FMT>(cur[k], xr[k], sx[k]);
                if (GROUPED) acc = fmaf(part, a.scales[vl * a.groups + lh_group_of(a, j * R)], acc);
                else acc += part;
            }
        }
        // the L partial sums of the row, in the VALU: an inclusive DPP scan
        // inside each 16-lane row (L = 16) or over the wave (L = 64), the
        // row's sum landing in its last lane (fixed order, deterministic)
        if (log2L == 4) {
            acc += __uint_as_float(dpp0<0x111>(__float_as_uint(acc)));
            acc += __uint_as_float(dpp0<0x112>(__float_as_uint(acc)));
            acc += __uint_as_float(dpp0<0x114>(__float_as_uint(acc)));
            acc += __uint_as_float(dpp0<0x118>(__float_as_uint(acc)));
        } else {
            acc = wscan_f32(acc);
        }
        if (li == L - 1 && v < a.V) {
            if (FMT != kLhF32 && !GROUPED) acc *= a.scales[v];  // dot * scale (quant.rs:128)
            if (!GREEDY || a.out != nullptr) a.out[v] = acc;
            if (GREEDY) {
                const unsigned long long k = lh_greedy_key(acc, v);
                best = k > best ? k : best;
            }
        }
    }
    if constexpr (GREEDY) {
        best = lh_wave_max_u64(best);
        if (lane == 0) gk[threadIdx.x >> 6] = best;
        __syncthreads();  // (waves past V took the same barrier)
        if (threadIdx.x == 0) a.part[blockIdx.x] = max(max(gk[0], gk[1]), max(gk[2], gk[3]));
    }
}

// The greedy token from n workgroup keys: one workgroup of 1024 lanes.
__global__ __launch_bounds__(1024) void lm_head_greedy_final_kernel(const unsigned long long* part,
                                                                    int n, uint32_t* token) {
    __shared__ unsigned long long wk[16];
    unsigned long long k = 0ull;
    for (int i = (int)threadIdx.x; i < n; i += 1024) k = part[i] > k ? part[i] : k;
    k = lh_wave_max_u64(k);
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x < 64) {
        unsigned long long t = threadIdx.x < 16 ? wk[threadIdx.x] : 0ull;
        t = lh_wave_max_u64(t);
        if (threadIdx.x == 0) *token = 0xFFFFFFFFu - (uint32_t)t;
    }
}


}  // namespace nis
