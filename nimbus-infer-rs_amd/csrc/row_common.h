// row_common.h — pieces every row kernel shares: the float4 vector types,
// the raw buffer load, LDS-only barriers and fences, masked LDS stores, and
// the fix-up of a row's partial head / tail float4 slots.
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

__device__ __forceinline__ float elem(const f4v& v, int q) {
    return q == 0 ? v.x : (q == 1 ? v.y : (q == 2 ? v.z : v.w));
}
__device__ __forceinline__ float max4(const f4v& v) {
    return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
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

// A 4-byte and a 1-byte LDS store by the lanes of `mask` only (as above).
__device__ __forceinline__ void lds_put_f32_u8(uint64_t mask, uint32_t a, float v, uint32_t b,
                                               uint32_t h) {
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %1\n\t"
        "ds_write_b32 %2, %3\n\t"
        "ds_write_b8 %4, %5\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(sv)
        : "s"(mask), "v"(a), "v"(v), "v"(b), "v"(h)
        : "memory");
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

}  // namespace nis
