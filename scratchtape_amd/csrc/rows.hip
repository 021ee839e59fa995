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
// column sums in two passes, each in a fixed order, on one of two paths:
//  - scalar path (any d, offset or alignment): k_ln_bwd_part sums 128-row
//    chunks (4 row lanes per column, combined in a fixed order) and
//    k_ln_bwd_sum adds the chunks in ascending order;
//  - vector path (d % 4 == 0 up to 1024, 16-byte aligned rows and parameter
//    sets): k_ln_bwd4 sums 16-row chunks (each of 4 waves adds its rows in
//    row order; the 4 waves' sums are added in wave order) and
//    k_ln_bwd_sum4 adds a column's chunks as 16 slices, each slice's chunks
//    in ascending order, the 16 slice sums in a fixed tree order.
// The two paths add in different orders, so their last bits can differ;
// each is deterministic.  Contraction is off so that scale*x - m rounds the
// product first, as the reference's CPU tape does.
#include "common.h"
#include "lanes.h"

#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ float wave_max(float v) {
    const int lane = st::lane_id();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, st::xor_lane(v, o, lane));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    const int lane = st::lane_id();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += st::xor_lane(v, o, lane);
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

// ---- Vector forms for rows of d % 4 == 0 up to 1024 wide, 16-byte aligned:
// lane l of a row's wave owns the float4 columns 4 l + 256 i, i < NV.

constexpr int LNV_ROWS = 16;  // rows per backward workgroup (4 per wave)

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
// Output rows (y, dx) through nontemporal stores: they stream out as the
// waves finish instead of waiting in L2 for the end-of-kernel write-back.
typedef float lnf4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st4(float *p, float4 v) {
    __builtin_nontemporal_store(lnf4{v.x, v.y, v.z, v.w}, reinterpret_cast<lnf4 *>(p));
}

// grid: ceil(rows / 4) workgroups of 4 row-waves.  The formulas of k_ln_fwd;
// a lane adds its four columns pairwise before the butterfly, so the row sums
// are in another (fixed) order.
template <int NV>
__global__ __launch_bounds__(256) void k_ln_fwd4(const float *__restrict__ x, int64_t rows, int64_t d,
                                                 const float *__restrict__ params, int64_t off, float eps,
                                                 int64_t rows_pm, int64_t stride, float *__restrict__ y,
                                                 float *__restrict__ mean, float *__restrict__ rstd) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *xr = x + r * d;
    const float *gm = params + off + (r / rows_pm) * stride, *bt = gm + d;
    float4 xv[NV], gv[NV], bv[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = 4 * lane + 256 * i;
        const bool in = j < d;
        xv[i] = in ? ld4(xr + j) : make_float4(0.f, 0.f, 0.f, 0.f);
        gv[i] = in ? ld4(gm + j) : make_float4(0.f, 0.f, 0.f, 0.f);
        bv[i] = in ? ld4(bt + j) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float inv_d = 1.0f / (float)d;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) s += ((xv[i].x + xv[i].y) + (xv[i].z + xv[i].w));
    const float mu = wave_sum(s) * inv_d;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        if (4 * lane + 256 * i < d) {
            const float a = xv[i].x - mu, b = xv[i].y - mu, c = xv[i].z - mu, e = xv[i].w - mu;
            sq += ((a * a + b * b) + (c * c + e * e));
        }
    }
    const float sd = sqrtf(wave_sum(sq) * inv_d + eps);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = 4 * lane + 256 * i;
        if (j < d) {
            float4 o;
            o.x = ((xv[i].x - mu) / sd) * gv[i].x + bv[i].x;
            o.y = ((xv[i].y - mu) / sd) * gv[i].y + bv[i].y;
            o.z = ((xv[i].z - mu) / sd) * gv[i].z + bv[i].z;
            o.w = ((xv[i].w - mu) / sd) * gv[i].w + bv[i].w;
            st4(y + r * d + j, o);
        }
    }
    if (lane == 0) {
        mean[r] = mu;
        rstd[r] = 1.0f / sd;
    }
}

// The backward's row pass.  grid (chunks of LNV_ROWS rows per model, models);
// wave w takes rows w, w + 4, .. of its chunk: dx as k_ln_bwd_dx, and each
// lane adds dy xhat and dy of its columns over the wave's rows (in row order).
// The four waves' sums are added in a fixed order into the chunk's partial,
// part[(m nch + c) 2d + j], which k_ln_bwd_sum4 adds up.  dy and x are read
// once for both gradients.
template <int NV>
__global__ __launch_bounds__(256) void k_ln_bwd4(const float *__restrict__ dy, const float *__restrict__ x,
                                                 const float *__restrict__ mean, const float *__restrict__ rstd,
                                                 int64_t d, int64_t rows_pm, const float *__restrict__ params,
                                                 int64_t off, int64_t stride, float *__restrict__ dx, int32_t accumulate,
                                                 float *__restrict__ part, int32_t nch) {
    __shared__ float4 sp[4][2][NV * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t c = blockIdx.x, m = blockIdx.y;
    const int64_t rbeg = (int64_t)m * rows_pm + (int64_t)c * LNV_ROWS;
    const int64_t rend = min((int64_t)m * rows_pm + rows_pm, rbeg + LNV_ROWS);
    const float *gm = params + off + (int64_t)m * stride;
    const float inv_d = 1.0f / (float)d;
    float4 gmv[NV], pg[NV], pb[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = 4 * lane + 256 * i;
        gmv[i] = j < d ? ld4(gm + j) : make_float4(0.f, 0.f, 0.f, 0.f);
        pg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        pb[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // RB rows' loads in flight together; a row past the chunk's end loads the
    // chunk's last row (always in bounds) and contributes nothing.
    constexpr int RB = NV >= 4 ? 2 : 4;
#pragma unroll
    for (int t0 = 0; t0 < LNV_ROWS / 4; t0 += RB) {
        float4 dyv[RB][NV], xv[RB][NV];
        float mu[RB], rs[RB];
        bool live[RB];
#pragma unroll
        for (int t = 0; t < RB; t++) {
            const int64_t r = rbeg + wave + 4 * (t0 + t);
            live[t] = r < rend;
            const int64_t rl = live[t] ? r : rend - 1;
            mu[t] = mean[rl];
            rs[t] = rstd[rl];
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int j = 4 * lane + 256 * i;
                const bool in = j < d;
                dyv[t][i] = in ? ld4(dy + rl * d + j) : make_float4(0.f, 0.f, 0.f, 0.f);
                xv[t][i] = in ? ld4(x + rl * d + j) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int t = 0; t < RB; t++) {
            if (!live[t]) break;
            const int64_t r = rbeg + wave + 4 * (t0 + t);
            float4 g[NV], h[NV];
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const bool in = 4 * lane + 256 * i < d;
                const float4 dv = dyv[t][i], xq = xv[t][i];
                const float m_ = mu[t], r_ = rs[t];
                g[i] = make_float4(dv.x * gmv[i].x, dv.y * gmv[i].y, dv.z * gmv[i].z, dv.w * gmv[i].w);
                h[i] = in ? make_float4((xq.x - m_) * r_, (xq.y - m_) * r_, (xq.z - m_) * r_, (xq.w - m_) * r_)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
                s1 += ((g[i].x + g[i].y) + (g[i].z + g[i].w));
                s2 += ((g[i].x * h[i].x + g[i].y * h[i].y) + (g[i].z * h[i].z + g[i].w * h[i].w));
            }
            s1 = wave_sum(s1) * inv_d;
            s2 = wave_sum(s2) * inv_d;
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int j = 4 * lane + 256 * i;
                const float r_ = rs[t];
                if (j < d) {
                    float4 v;
                    v.x = r_ * (g[i].x - s1 - h[i].x * s2);
                    v.y = r_ * (g[i].y - s1 - h[i].y * s2);
                    v.z = r_ * (g[i].z - s1 - h[i].z * s2);
                    v.w = r_ * (g[i].w - s1 - h[i].w * s2);
                    if (accumulate) {
                        const float4 o = ld4(dx + r * d + j);
                        v.x = o.x + v.x;
                        v.y = o.y + v.y;
                        v.z = o.z + v.z;
                        v.w = o.w + v.w;
                    }
                    st4(dx + r * d + j, v);
                }
                const float4 dv = dyv[t][i];
                pg[i].x += dv.x * h[i].x;
                pg[i].y += dv.y * h[i].y;
                pg[i].z += dv.z * h[i].z;
                pg[i].w += dv.w * h[i].w;
                pb[i].x += dv.x;
                pb[i].y += dv.y;
                pb[i].z += dv.z;
                pb[i].w += dv.w;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
        sp[wave][0][64 * i + lane] = pg[i];
        sp[wave][1][64 * i + lane] = pb[i];
    }
    __syncthreads();
    // Column j of the chunk partial (j < d: dgamma, d <= j < 2d: dbeta).
    const float *spf = reinterpret_cast<const float *>(sp);
    constexpr int HALF = NV * 256, WSTRIDE = 2 * HALF;  // floats per half, per wave
    float *pc = part + ((int64_t)m * nch + c) * 2 * d;
    for (int j = tid; j < 2 * d; j += 256) {
        const int o = (j < d ? j : HALF + (j - d));
        pc[j] = (spf[o] + spf[WSTRIDE + o]) + (spf[2 * WSTRIDE + o] + spf[3 * WSTRIDE + o]);
    }
}

// grid (ceil(2d / 16), models): grads[off + m stride + j] += the sum over the
// nch chunk partials of column j.  Thread (slice sl, column tx) adds chunks
// sl per .. (sl + 1) per - 1 in order (sixteen loads in flight at a time), and
// the sixteen slices' sums are added in a fixed tree order.
__global__ __launch_bounds__(256) void k_ln_bwd_sum4(const float *__restrict__ part, int64_t d, int32_t nch,
                                                     float *__restrict__ grads, int64_t off, int64_t stride) {
    __shared__ float red[16][17];
    const int tx = threadIdx.x & 15, sl = threadIdx.x >> 4;
    const int64_t j = (int64_t)blockIdx.x * 16 + tx, m = blockIdx.y;
    const int32_t per = (nch + 15) / 16, c0 = sl * per, c1 = min(nch, c0 + per);
    float sum = 0.f;
    if (j < 2 * d) {
        for (int32_t c = c0; c < c1; c += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = c + u < c1 ? part[((int64_t)m * nch + c + u) * 2 * d + j] : 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (c + u < c1) sum += v[u];
        }
    }
    red[sl][tx] = sum;
    __syncthreads();
#pragma unroll
    for (int w = 8; w > 0; w >>= 1) {
        if (sl < w) red[sl][tx] = red[sl][tx] + red[sl + w][tx];
        __syncthreads();
    }
    if (sl == 0 && j < 2 * d) grads[off + m * stride + j] += red[0][tx];
}

// Whether the vector forms apply: d % 4 == 0 up to 1024, every row and
// parameter set 16-byte aligned.
bool ln_vec_ok(int64_t d, int64_t off, int64_t stride, std::initializer_list<const void *> ptrs) {
    if (d % 4 != 0 || d > 1024 || off % 4 != 0 || stride % 4 != 0) return false;
    for (const void *p : ptrs)
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    return true;
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
    const dim3 grid((unsigned)((rows + 3) / 4));
    const hipStream_t s = st::stream_of(stream);
    const int64_t rows_pm = rows / models;
    if (ln_vec_ok(d, off, model_stride, {x, params, y})) {
        const int nv = (int)((d + 255) / 256);
        auto k = nv == 1 ? k_ln_fwd4<1> : nv == 2 ? k_ln_fwd4<2> : k_ln_fwd4<4>;
        hipLaunchKernelGGL(k, grid, dim3(256), 0, s, x, rows, d, params, off, eps, rows_pm, model_stride, y, mean,
                           rstd);
    } else {
        hipLaunchKernelGGL(k_ln_fwd, grid, dim3(256), 0, s, x, rows, d, params, off, eps, rows_pm, model_stride, y,
                           mean, rstd);
    }
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
    const int64_t rows_pm = rows / models;
    const int64_t vch = (rows_pm + LNV_ROWS - 1) / LNV_ROWS;
    if (ln_vec_ok(d, off, model_stride, {dy, x, params, dx}) && vch <= INT32_MAX && models <= 65535) {
        float *part = static_cast<float *>(
            st::scratch(st::SCRATCH_ROWS, (size_t)(models * vch * 2 * d) * sizeof(float), s));
        if (!part) return st::scratch_status();
        const int nv = (int)((d + 255) / 256);
        auto k = nv == 1 ? k_ln_bwd4<1> : nv == 2 ? k_ln_bwd4<2> : k_ln_bwd4<4>;
        hipLaunchKernelGGL(k, dim3((unsigned)vch, (unsigned)models), dim3(256), 0, s, dy, x, mean, rstd, d, rows_pm,
                           params, off, model_stride, dx, accumulate, part, (int32_t)vch);
        ST_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_ln_bwd_sum4, dim3((unsigned)((2 * d + 15) / 16), (unsigned)models), dim3(256), 0, s, part,
                           d, (int32_t)vch, grads, off, model_stride);
        ST_LAUNCH_CHECK();
        return ST_OK;
    }
    const int64_t nch = (rows_pm + LN_CHUNK - 1) / LN_CHUNK;
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
