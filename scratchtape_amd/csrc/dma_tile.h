// Device helpers shared by the LDS-DMA GEMM kernels (gemm_dma.hip: one GEMM
// per launch; gemm_group.hip: several independent GEMMs in one persistent
// launch): the global -> LDS DMA of 16 bytes per lane, explicit vmcnt waits,
// a fence-free workgroup barrier, and the two LDS layouts of a 32-deep
// k-stage of an f32 operand tile.
//
//  - KC, an operand whose k is contiguous in memory (A not transposed, B
//    transposed): [row][8 chunks of 4 k]; chunk c of row r sits in slot
//    r * 8 + (c ^ ((r >> 1) & 7)).  A fragment (8 k of one row per lane) is two
//    128-bit reads; the swizzle puts the 16 rows a quarter-wave reads in 16
//    distinct 16-byte bank groups.
//  - RC, an operand whose rows are contiguous (A transposed, B not): [k][rows],
//    line kk holding rows in chunks of 4 rotated by 16 rows per group of 8 k:
//    chunk q of line kk sits in slot kk * Q + (q + 4 * ((kk >> 3) & 3)) % Q,
//    Q = ROWS / 4.  A fragment is eight 32-bit reads; the 64 lanes of each read
//    hit 64 distinct banks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dma {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 32;  // k per stage

// 16 bytes per lane from global memory to LDS: lane l's 16 bytes from gptr
// land at LDS byte address lds_addr + 16 l (lds_addr wave-uniform, passed in
// M0).  Issued as inline assembly so that the compiler sees no LDS store in
// flight: it would otherwise wait for every DMA before each LDS read (it cannot
// tell which stage a DMA writes).  Completion is tracked by explicit vmcnt
// waits, followed by a workgroup barrier, before any wave reads the stage.  M0
// is saved and restored around the load, so the compiler's view of it stays
// valid, and one wait state separates the M0 write from the LDS DMA that reads
// it (a gfx9 hazard the compiler does not guard in inline asm).
__device__ __forceinline__ void dma16(const float *gptr, uint32_t lds_addr) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(gptr), "s"(lds_addr)
        : "memory");
}

// One k-stage's DMA of one wave for the grouped GEMM: LA loads of operand A
// from abase + ao[i] into LDS m0a + 1024 i, then LB of B from bbase + bo[i]
// into m0b + 1024 i (bases wave-uniform in SGPRs, per-lane byte offsets in
// VGPRs).  The instruction offset 1024 i is added to both the global and the
// LDS address, so ao[i] / bo[i] are the source offsets minus 1024 i and M0 is
// written once per operand; one wait state separates each M0 write from the
// loads that read it, and M0 is restored at the end.
template <int LA, int LB>
__device__ __forceinline__ void dma_stage(const void *abase, const uint32_t (&ao)[LA], uint32_t m0a,
                                          const void *bbase, const uint32_t (&bo)[LB], uint32_t m0b);

template <>
__device__ __forceinline__ void dma_stage<4, 4>(const void *abase, const uint32_t (&ao)[4], uint32_t m0a,
                                                const void *bbase, const uint32_t (&bo)[4], uint32_t m0b) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %9\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %10\n\t"
        "global_load_lds_dwordx4 %2, %10 offset:1024\n\t"
        "global_load_lds_dwordx4 %3, %10 offset:2048\n\t"
        "global_load_lds_dwordx4 %4, %10 offset:3072\n\t"
        "s_mov_b32 m0, %11\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %5, %12\n\t"
        "global_load_lds_dwordx4 %6, %12 offset:1024\n\t"
        "global_load_lds_dwordx4 %7, %12 offset:2048\n\t"
        "global_load_lds_dwordx4 %8, %12 offset:3072\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(ao[0]), "v"(ao[1]), "v"(ao[2]), "v"(ao[3]), "v"(bo[0]), "v"(bo[1]), "v"(bo[2]), "v"(bo[3]), "s"(m0a),
          "s"(abase), "s"(m0b), "s"(bbase)
        : "memory");
}

template <>
__device__ __forceinline__ void dma_stage<4, 2>(const void *abase, const uint32_t (&ao)[4], uint32_t m0a,
                                                const void *bbase, const uint32_t (&bo)[2], uint32_t m0b) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %7\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %8\n\t"
        "global_load_lds_dwordx4 %2, %8 offset:1024\n\t"
        "global_load_lds_dwordx4 %3, %8 offset:2048\n\t"
        "global_load_lds_dwordx4 %4, %8 offset:3072\n\t"
        "s_mov_b32 m0, %9\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %5, %10\n\t"
        "global_load_lds_dwordx4 %6, %10 offset:1024\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(ao[0]), "v"(ao[1]), "v"(ao[2]), "v"(ao[3]), "v"(bo[0]), "v"(bo[1]), "s"(m0a), "s"(abase), "s"(m0b),
          "s"(bbase)
        : "memory");
}

__device__ __forceinline__ uint32_t lds_addr_of(const float *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)p;
}

// Waits until at most N vector-memory instructions of this wave are in flight
// (they complete in issue order, loads and stores alike).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waits until this wave's DMA of the oldest stage in flight has landed, with
// `ahead` (0 .. MAXA) younger stages of L instructions each still in flight.
// Other vector-memory instructions issued after that stage only make the wait
// longer, never too short.
template <int L, int MAXA>
__device__ __forceinline__ void wait_stage(int ahead) {
    if constexpr (MAXA >= 4) {
        if (ahead >= 4) return wait_vm<4 * L>();
    }
    if constexpr (MAXA >= 3) {
        if (ahead == 3) return wait_vm<3 * L>();
    }
    if constexpr (MAXA >= 2) {
        if (ahead == 2) return wait_vm<2 * L>();
    }
    if constexpr (MAXA >= 1) {
        if (ahead == 1) return wait_vm<L>();
    }
    wait_vm<0>();
}

// Workgroup barrier without the memory fence of __syncthreads() (which would
// wait for every load of this wave, the DMA of the younger stages included);
// the empty asm statements keep the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void bar() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Element offset (from the operand's matrix base, at k = 0) of the 16 bytes
// that DMA slot p of a ROWS x 32 stage tile receives.
template <int ROWS, bool KC>
__device__ __forceinline__ int64_t slot_src(int p, int64_t ld, int row0) {
    if constexpr (KC) {
        const int r = p >> 3, c = (p & 7) ^ ((r >> 1) & 7);
        return (int64_t)(row0 + r) * ld + 4 * c;
    } else {
        constexpr int Q = ROWS / 4;
        const int kk = p / Q, s = p % Q;
        const int q = (s - 4 * ((kk >> 3) & 3) + 4 * Q) % Q;
        return (int64_t)kk * ld + row0 + 4 * q;
    }
}

// The 8 values (k = 8g .. 8g + 7 of the stage) of row r of a stage tile.
template <int ROWS, bool KC>
__device__ __forceinline__ void frag(const float *t, int r, int g, float (&x)[8]) {
    if constexpr (KC) {
        const int sw = (r >> 1) & 7;
        const f32x4 lo = *reinterpret_cast<const f32x4 *>(t + (r * 8 + ((2 * g) ^ sw)) * 4);
        const f32x4 hi = *reinterpret_cast<const f32x4 *>(t + (r * 8 + ((2 * g + 1) ^ sw)) * 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[e] = lo[e];
            x[4 + e] = hi[e];
        }
    } else {
        constexpr int Q = ROWS / 4;
        const int q = ((r >> 2) + 4 * g) % Q;  // (kk >> 3) & 3 == g for kk = 8g + u
#pragma unroll
        for (int u = 0; u < 8; u++) x[u] = t[((8 * g + u) * Q + q) * 4 + (r & 3)];
    }
}

// acc + src[0] + src[step] + .. + src[(splits - 1) step], added in that order
// (the deterministic split-k sum), with the loads of up to 16 slices issued
// before the first add: one memory round trip per 16 slices, not one per slice.
template <class P, class T>
__device__ __forceinline__ T sum_slices(P src, int64_t step, int splits, T acc) {
    for (int s0 = 0; s0 < splits; s0 += 16) {
        T v[16];
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (s0 + j < splits) v[j] = src[(s0 + j) * step];
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (s0 + j < splits) acc += v[j];
    }
    return acc;
}

__device__ __forceinline__ int64_t zoff(int64_t z, int64_t group, int64_t stride, int64_t inner) {
    return (z / group) * stride + (z % group) * inner;
}

}  // namespace dma
