// Row-wise kernels beside the GEMMs: causal softmax and its backward for the
// attention configuration, LayerNorm forward and backward.
//
// Reference semantics: gpu_step/rows.rs:101-123 (softmax, softmax_backward)
// and the kernels k_softmax_fwd / k_softmax_bwd (rows.rs:295-357): row r of
// x [rows, n] is query position r % t and sees columns 0..=r % t; masked
// entries are exactly 0; softmax1 adds a phantom logit 0 with the shift
// max(row max, 0).
//
// LayerNorm (gpu_step/rows.rs:60-99 layer_norm / layer_norm_backward and
// k_ln_fwd, k_ln_bwd_dx, k_ln_bwd_params rows.rs:177-293; nn.rs:306-321 on the
// CPU tape): y = (x - mean) / sqrt(var + eps) * gamma + beta per row, biased
// variance; dx (+)= rstd (g - mean(g) - xhat mean(g xhat)), g = dy gamma;
// gamma / beta gradients accumulate as column sums over each model's rows.
//
// One wave64 per row (4 rows per 256-thread workgroup); each lane walks the
// row with stride 64, and the row max / sum are fixed butterfly reductions
// over the wave, so results are deterministic.  The parameter gradients are
// column sums in two passes: partial sums over 128-row chunks (4 row lanes
// per column, combined in a fixed order), then the chunks summed in order.  Contraction is off so that
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

constexpr int LN_CHUNK = 128;  // rows per partial column sum
constexpr int LN_REG = 16;     // row values held per lane (rows up to 1024 wide read once)

// grid: ceil(rows / 4) workgroups of 4 row-waves.
__global__ __launch_bounds__(256) void k_ln_fwd(const float *__restrict__ x, int64_t rows, int64_t d,
                                                const float *__restrict__ params, int64_t off, float eps,
                                                int64_t rows_pm, int64_t stride, float *__restrict__ y,
                                                float *__restrict__ mean, float *__restrict__ rstd) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *xr = x + r * d;
    const float *gm = params + off + (r / rows_pm) * stride, *bt = gm + d;
    const float inv_d = 1.0f / (float)d;
    // Rows of up to 1024 columns are held in registers (16 per lane), so the
    // row is read from memory once; wider rows re-read it.
    float xv[LN_REG];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < LN_REG; i++) {
        const int64_t j = lane + 64 * i;
        xv[i] = j < d ? xr[j] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < LN_REG; i++)
        if (lane + 64 * i < d) s += xv[i];
    for (int64_t j = lane + 64 * LN_REG; j < d; j += 64) s += xr[j];
    const float mu = wave_sum(s) * inv_d;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < LN_REG; i++) {
        if (lane + 64 * i < d) {
            const float c = xv[i] - mu;
            sq += c * c;
        }
    }
    for (int64_t j = lane + 64 * LN_REG; j < d; j += 64) {
        const float c = xr[j] - mu;
        sq += c * c;
    }
    const float sd = sqrtf(wave_sum(sq) * inv_d + eps);
#pragma unroll
    for (int i = 0; i < LN_REG; i++) {
        const int64_t j = lane + 64 * i;
        if (j < d) y[r * d + j] = ((xv[i] - mu) / sd) * gm[j] + bt[j];
    }
    for (int64_t j = lane + 64 * LN_REG; j < d; j += 64) y[r * d + j] = ((xr[j] - mu) / sd) * gm[j] + bt[j];
    if (lane == 0) {
        mean[r] = mu;
        rstd[r] = 1.0f / sd;
    }
}

__global__ __launch_bounds__(256) void k_ln_bwd_dx(const float *__restrict__ dy, const float *__restrict__ x,
                                                   const float *__restrict__ mean, const float *__restrict__ rstd,
                                                   int64_t rows, int64_t d, const float *__restrict__ params,
                                                   int64_t off, float *__restrict__ dx, int32_t accumulate,
                                                   int64_t rows_pm, int64_t stride) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *gm = params + off + (r / rows_pm) * stride;
    const float mu = mean[r], rs = rstd[r];
    const int64_t base = r * d;
    float gv[LN_REG], hv[LN_REG];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < LN_REG; i++) {
        const int64_t j = lane + 64 * i;
        gv[i] = j < d ? dy[base + j] * gm[j] : 0.f;
        hv[i] = j < d ? (x[base + j] - mu) * rs : 0.f;
    }
#pragma unroll
    for (int i = 0; i < LN_REG; i++) {
        if (lane + 64 * i < d) {
            s1 += gv[i];
            s2 += gv[i] * hv[i];
        }
    }
    for (int64_t j = lane + 64 * LN_REG; j < d; j += 64) {
        const float g = dy[base + j] * gm[j];
        s1 += g;
        s2 += g * ((x[base + j] - mu) * rs);
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float inv_d = 1.0f / (float)d;
#pragma unroll
    for (int i = 0; i < LN_REG; i++) {
        const int64_t j = lane + 64 * i;
        if (j < d) {
            const float v = rs * (gv[i] - s1 * inv_d - hv[i] * (s2 * inv_d));
            dx[base + j] = accumulate ? dx[base + j] + v : v;
        }
    }
    for (int64_t j = lane + 64 * LN_REG; j < d; j += 64) {
        const float g = dy[base + j] * gm[j];
        const float xh = (x[base + j] - mu) * rs;
        const float v = rs * (g - s1 * inv_d - xh * (s2 * inv_d));
        dx[base + j] = accumulate ? dx[base + j] + v : v;
    }
}

// grid (ceil(d / 64) column blocks, chunks per model, models): part[(m nch + c)
// 2d + j] = sum of dy xhat over the chunk's rows of column j, + d: of dy.
__global__ __launch_bounds__(256) void k_ln_bwd_part(const float *__restrict__ dy, const float *__restrict__ x,
                                                     const float *__restrict__ mean, const float *__restrict__ rstd,
                                                     int64_t d, int64_t rows_pm, float *__restrict__ part) {
    __shared__ float sg[4][64], sb[4][64];
    const int tx = threadIdx.x & 63, lane = threadIdx.x >> 6;
    const int64_t j = (int64_t)blockIdx.x * 64 + tx;
    const int64_t c = blockIdx.y, m = blockIdx.z, nch = gridDim.y;
    const int64_t r0 = m * rows_pm + c * LN_CHUNK;
    const int64_t r1 = min(m * rows_pm + rows_pm, r0 + LN_CHUNK);
    float pg = 0.f, pb = 0.f;
    if (j < d) {
#pragma unroll 4
        for (int64_t r = r0 + lane; r < r1; r += 4) {
            const float g = dy[r * d + j];
            pg += g * ((x[r * d + j] - mean[r]) * rstd[r]);
            pb += g;
        }
    }
    sg[lane][tx] = pg;
    sb[lane][tx] = pb;
    __syncthreads();
    if (lane == 0 && j < d) {
        float *pp = part + (m * nch + c) * 2 * d;
        pp[j] = (sg[0][tx] + sg[1][tx]) + (sg[2][tx] + sg[3][tx]);
        pp[d + j] = (sb[0][tx] + sb[1][tx]) + (sb[2][tx] + sb[3][tx]);
    }
}

// grid (ceil(2d / 256), models): grads[off + m stride + j] += the chunks' partials in order.
__global__ __launch_bounds__(256) void k_ln_bwd_sum(const float *__restrict__ part, int64_t d, int64_t nch,
                                                    float *__restrict__ grads, int64_t off, int64_t stride) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
    if (j >= 2 * d) return;
    float s = 0.f;
    int64_t c = 0;
    for (; c + 8 <= nch; c += 8) {  // eight loads in flight, added in chunk order
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = part[(m * nch + c + u) * 2 * d + j];
#pragma unroll
        for (int u = 0; u < 8; u++) s += v[u];
    }
    for (; c < nch; c++) s += part[(m * nch + c) * 2 * d + j];
    grads[off + m * stride + j] += s;
}

st_status ln_check(const char *what, int64_t rows, int64_t d, int64_t off, int64_t models, int64_t stride) {
    if (rows < 0 || d < 1 || off < 0) return st::fail(ST_ERR_INVALID, "%s: bad rows, d or offset", what);
    if (models < 1 || rows % models != 0)
        return st::fail(ST_ERR_INVALID, "%s: rows (%lld) must split evenly over %lld models", what, (long long)rows,
                        (long long)models);
    if (models > 1 && stride < 2 * d)
        return st::fail(ST_ERR_INVALID, "%s: models' parameter sets overlap (stride %lld < 2 d)", what,
                        (long long)stride);
    if ((rows + 3) / 4 > INT32_MAX) return st::fail(ST_ERR_INVALID, "%s: too many rows", what);
    return ST_OK;
}

}  // namespace

extern "C" st_status st_layer_norm(const float *x, int64_t rows, int64_t d, const float *params, int64_t off,
                                   float eps, int64_t models, int64_t model_stride, float *y, float *mean,
                                   float *rstd, st_stream stream) {
    st::clear_error();
    if (!x || !params || !y || !mean || !rstd) return st::fail(ST_ERR_INVALID, "layer_norm: NULL buffer");
    st_status st = ln_check("layer_norm", rows, d, off, models, model_stride);
    if (st != ST_OK || rows == 0) return st;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    hipLaunchKernelGGL(k_ln_fwd, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st::stream_of(stream), x, rows, d,
                       params, off, eps, rows / models, model_stride, y, mean, rstd);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_layer_norm_backward(const float *dy, const float *x, const float *mean, const float *rstd,
                                            int64_t rows, int64_t d, const float *params, float *grads,
                                            int64_t off, float *dx, int32_t accumulate, int64_t models,
                                            int64_t model_stride, st_stream stream) {
    st::clear_error();
    if (!dy || !x || !mean || !rstd || !params || !grads || !dx)
        return st::fail(ST_ERR_INVALID, "layer_norm_backward: NULL buffer");
    st_status st = ln_check("layer_norm_backward", rows, d, off, models, model_stride);
    if (st != ST_OK || rows == 0) return st;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const hipStream_t s = st::stream_of(stream);
    const int64_t rows_pm = rows / models, nch = (rows_pm + LN_CHUNK - 1) / LN_CHUNK;
    if (nch > 65535 || models > 65535 || (d + 63) / 64 > INT32_MAX)
        return st::fail(ST_ERR_INVALID, "layer_norm_backward: too many rows per model or models");
    float *part = static_cast<float *>(st::scratch(st::SCRATCH_ROWS, (size_t)(models * nch * 2 * d) * sizeof(float), s));
    if (!part) return st::scratch_status();
    hipLaunchKernelGGL(k_ln_bwd_dx, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, dy, x, mean, rstd, rows, d,
                       params, off, dx, accumulate, rows_pm, model_stride);
    ST_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_ln_bwd_part, dim3((unsigned)((d + 63) / 64), (unsigned)nch, (unsigned)models), dim3(256), 0,
                       s, dy, x, mean, rstd, d, rows_pm, part);
    ST_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_ln_bwd_sum, dim3((unsigned)((2 * d + 255) / 256), (unsigned)models), dim3(256), 0, s, part,
                       d, nch, grads, off, model_stride);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

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
