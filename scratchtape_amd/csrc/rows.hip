// Row-wise causal softmax and its backward for the attention configuration.
//
// Reference semantics: gpu_step/rows.rs:101-123 (softmax, softmax_backward)
// and the kernels k_softmax_fwd / k_softmax_bwd (rows.rs:295-357): row r of
// x [rows, n] is query position r % t and sees columns 0..=r % t; masked
// entries are exactly 0; softmax1 adds a phantom logit 0 with the shift
// max(row max, 0).
//
// One wave64 per row (4 rows per 256-thread workgroup); each lane walks the
// row with stride 64, and the row max / sum are fixed butterfly reductions
// over the wave, so results are deterministic.  Contraction is off so that
// scale*x - m rounds the product first, as the reference's CPU tape does.
#include "common.h"

#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__global__ __launch_bounds__(256) void k_softmax_fwd(const float *__restrict__ x, float *__restrict__ y,
                                                     int64_t rows, int64_t n, int64_t t, float scale,
                                                     int32_t causal, int32_t one) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *xr = x + r * n;
    float *yr = y + r * n;
    int64_t limit = causal ? (r % t) + 1 : n;
    if (limit > n) limit = n;
    // Column 0 is always visible, so every lane's max starts from it.
    float m = scale * xr[0];
    for (int64_t j = lane; j < limit; j += 64) m = fmaxf(m, scale * xr[j]);
    m = wave_max(m);
    if (one && m < 0.f) m = 0.f;
    float s = 0.f;
    for (int64_t j = lane; j < limit; j += 64) s += expf(scale * xr[j] - m);
    s = wave_sum(s);
    if (one) s += expf(-m);
    for (int64_t j = lane; j < n; j += 64) yr[j] = j < limit ? expf(scale * xr[j] - m) / s : 0.f;
}

__global__ __launch_bounds__(256) void k_softmax_bwd(const float *__restrict__ dy, const float *__restrict__ y,
                                                     float *__restrict__ dx, int64_t rows, int64_t n, float scale) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int64_t base = r * n;
    float d = 0.f;
    for (int64_t j = lane; j < n; j += 64) d += dy[base + j] * y[base + j];
    d = wave_sum(d);
    for (int64_t j = lane; j < n; j += 64) dx[base + j] = scale * y[base + j] * (dy[base + j] - d);
}

}  // namespace

extern "C" st_status st_softmax(const float *x, float *y, int64_t rows, int64_t n, int64_t t, float scale,
                                int32_t causal, int32_t one, st_stream stream) {
    st::clear_error();
    if (!x || !y) return st::fail(ST_ERR_INVALID, "softmax: NULL buffer");
    if (rows < 0 || n < 0) return st::fail(ST_ERR_INVALID, "softmax: negative shape");
    if (causal && t <= 0) return st::fail(ST_ERR_INVALID, "softmax: causal needs t >= 1");
    if (rows == 0 || n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > INT32_MAX) return st::fail(ST_ERR_INVALID, "softmax: too many rows");
    hipLaunchKernelGGL(k_softmax_fwd, dim3((unsigned)blocks), dim3(256), 0, st::stream_of(stream), x, y, rows, n,
                       causal ? t : 1, scale, causal, one);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_softmax_backward(const float *dy, const float *y, float *dx, int64_t rows, int64_t n,
                                         float scale, st_stream stream) {
    st::clear_error();
    if (!dy || !y || !dx) return st::fail(ST_ERR_INVALID, "softmax_backward: NULL buffer");
    if (rows < 0 || n < 0) return st::fail(ST_ERR_INVALID, "softmax_backward: negative shape");
    if (rows == 0 || n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > INT32_MAX) return st::fail(ST_ERR_INVALID, "softmax_backward: too many rows");
    hipLaunchKernelGGL(k_softmax_bwd, dim3((unsigned)blocks), dim3(256), 0, st::stream_of(stream), dy, y, dx, rows,
                       n, scale);
    ST_LAUNCH_CHECK();
    return ST_OK;
}
