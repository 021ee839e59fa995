// Internal interface between the GEMM entry points (gemm.hip) and the
// LDS-DMA GEMM (gemm_dma.hip).
#pragma once

#include "common.h"

namespace st {

// One batched GEMM out[z] (+)= epi(a[z] @ b[z]); operand pointers already
// include their element offsets; z addresses a matrix as
// (z / group) * stride + (z % group) * inner.
struct DmaGemm {
    const float *a;
    int64_t a_stride, a_group, a_inner, lda;
    int32_t ta;
    const float *b;
    int64_t b_stride, b_group, b_inner, ldb;
    int32_t tb;
    float *out;
    int64_t o_stride, o_group, o_inner, ldo;
    const float *bias;  // + bias_off
    int64_t bias_stride;
    const float *mask;  // + mask_off
    const float *res;   // + residual_off
    float *cs;          // out buffer + col_sum_off
    int64_t cs_stride;
    int32_t has_cs, relu, accumulate;
    int32_t f16;
    int64_t batch, m, k, n;
};

// Enqueues the GEMM on the LDS-DMA kernel when the shape and alignment allow
// it (tile-divisible m and n, k % 32 == 0, 16-byte aligned operands and
// strides).  Returns false, having enqueued nothing, when they do not;
// otherwise true, with *status the launch status.
bool gemm_dma(const DmaGemm &g, hipStream_t stream, st_status *status);
// Whether gemm_dma takes g, and the bytes of split-k scratch it then requests
// (0 when it does not split).
bool gemm_dma_takes(const DmaGemm &g);
size_t gemm_dma_scratch(const DmaGemm &g);

// Grouped launches (gemm_group.hip): at most GROUP_MAX GEMMs of one route
// (f16 or f32) and one tile shape (group_tall: m % 256 == 0, 256-row tiles;
// else 128-row tiles) per launch, each of them group_eligible (m % 128 == 0,
// n % 128 == 0, k % 32 == 0, k >= 128, 16-byte aligned operands, strides and
// leading dimensions that fit the kernel's 32-bit fields).
constexpr int GROUP_MAX = 16;
bool group_eligible(const DmaGemm &g);
bool group_tall(const DmaGemm &g);
st_status gemm_group(const DmaGemm *items, int count, bool f16, bool tall, hipStream_t stream);
// Bytes of split-k scratch gemm_group requests for the same arguments.
size_t gemm_group_scratch(const DmaGemm *items, int count, bool f16, bool tall);
// Reads and clears the current device's count of grouped-kernel slot waits
// that gave up; ST_ERR_HIP with a message if there were any.  The caller has
// synchronised the work it wants covered.
st_status check_group_waits();

}  // namespace st
