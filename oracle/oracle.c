/*
 * CPU oracle for the scratchtape matrix-multiplication hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the reference
 * algorithms the HIP library must reproduce.  The parity tests and the
 * small-case check inside the package smoke run compare the library against
 * it, and the benchmark times it as the CPU baseline.  Nothing in the product library links,
 * loads or calls it.
 *
 * Build: gcc -O3 -mavx2 -mfma -ffp-contract=off -fopenmp -fPIC -shared (see
 * Makefile).  -ffp-contract=off matters: Rust never contracts a*b+c into an
 * FMA, so the restated loops must keep every multiply and add separately
 * rounded.
 *
 * Threads: orc_matmul, orc_transpose and orc_knn_search split their rows (or
 * queries) over orc_set_threads(n) OpenMP threads (1 by default, the
 * reference's single-threaded CPU path).  Each output element is computed by
 * one thread in the same order as with one, so the results do not depend on
 * the thread count; more threads only serve the all-cores CPU baseline.
 *
 * Pinning of every function (which test pins it and how) is listed in the
 * header comment of oracle/__init__.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 1;

void orc_set_threads(int32_t n) { g_threads = n < 1 ? 1 : n; }

int32_t orc_get_threads(void) { return g_threads; }

/* ------------------------------------------------------------------------ */
/* Rng: xorshift64 (13, 7, 17), src/nn.rs:8-35.                              */
/* ------------------------------------------------------------------------ */

/* Rng::next_f32, src/nn.rs:20-25: advance, then (state as f64 / u64::MAX as
 * f64) as f32.  u64 -> f64 and f64 -> f32 both round to nearest. */
float orc_rng_next_f32(uint64_t *s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return (float)((double)x / (double)UINT64_MAX);
}

/* Rng::next_gaussian, src/nn.rs:31-35: Box-Muller in f32, u1 floored at 1e-9. */
float orc_rng_next_gaussian(uint64_t *s) {
    float u1 = orc_rng_next_f32(s);
    if (!(u1 >= 1e-9f)) u1 = 1e-9f; /* f32::max(u1, 1e-9) */
    float u2 = orc_rng_next_f32(s);
    const float two_pi = 2.0f * 3.14159265358979323846f; /* 2.0 * consts::PI in f32 */
    float r = sqrtf(-2.0f * logf(u1));
    return r * cosf(two_pi * u2);
}

/* n values of next_f32()*2-1 (gpu.rs:189-192 input generator). */
void orc_rng_fill_uniform(uint64_t *s, int64_t n, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_rng_next_f32(s) * 2.0f - 1.0f;
}

/* n values of scale * next_gaussian() (scale 1: nn.rs:31-35 as used by the
 * reference tests; scale 0.02: the weight init of the step configuration). */
void orc_rng_fill_gaussian(uint64_t *s, int64_t n, float scale, float *out) {
    for (int64_t i = 0; i < n; i++) {
        float g = orc_rng_next_gaussian(s);
        out[i] = scale == 1.0f ? g : scale * g;
    }
}

/* ------------------------------------------------------------------------ */
/* NdArray::matmul / transpose, src/tensor.rs:241-287.                       */
/* ------------------------------------------------------------------------ */

/* tensor.rs:248-276: i and p blocked by 64, j full width, p ascending within
 * each (i, p-block); out[i*n+j] += a_ip * b[p*n+j] with a separately rounded
 * multiply and add. */
void orc_matmul(const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n) {
    const int64_t BLOCK = 64;
    memset(out, 0, sizeof(float) * (size_t)(m * n));
#pragma omp parallel for schedule(dynamic) num_threads(g_threads) if (g_threads > 1)
    for (int64_t i0 = 0; i0 < m; i0 += BLOCK) {
        int64_t i_max = i0 + BLOCK < m ? i0 + BLOCK : m;
        for (int64_t p0 = 0; p0 < k; p0 += BLOCK) {
            int64_t p_max = p0 + BLOCK < k ? p0 + BLOCK : k;
            for (int64_t i = i0; i < i_max; i++) {
                float *o = out + i * n;
                for (int64_t p = p0; p < p_max; p++) {
                    const float a_ip = a[i * k + p];
                    const float *bp = b + p * n;
                    for (int64_t j = 0; j < n; j++) o[j] += a_ip * bp[j];
                }
            }
        }
    }
}

/* tensor.rs:278-287: [m, n] -> [n, m]. */
void orc_transpose(const float *a, float *out, int64_t m, int64_t n) {
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1)
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) out[j * m + i] = a[i * n + j];
}

/* ------------------------------------------------------------------------ */
/* f32 <-> f16, round to nearest even (half 2.7.1 from_f32 / cubecl cast).   */
/* ------------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (ex == 0xffu) { /* inf or nan */
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int32_t e = (int32_t)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow */
    if (e <= 0) {
        /* subnormal half (or zero): value = man24 * 2^(ex-150), half ulp 2^-24 */
        if (e < -10) return (uint16_t)sign; /* below half of the smallest subnormal */
        uint32_t m24 = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e); /* bits to drop */
        uint32_t q = m24 >> shift;
        uint32_t rem = m24 & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry into exponent: correct */
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (ex == 0x1fu) {
        x = sign | 0x7f800000u | (man << 13);
    } else if (ex == 0) {
        if (man == 0) {
            x = sign;
        } else {
            float v = (float)man * 5.9604644775390625e-08f; /* man * 2^-24, exact */
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else {
        x = sign | ((ex - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

float orc_round_f16(float f) { return orc_f16_to_f32(orc_f32_to_f16(f)); }

void orc_round_f16_array(const float *in, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_round_f16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* gpu_step::matmul semantics: MatRef (matmul.rs:26-60) and Epilogue        */
/* (matmul.rs:62-79), as the plain-loop spec reference() (matmul.rs:888-937) */
/* with the head-view addressing of k_matmul (matmul.rs:374-378).            */
/* ------------------------------------------------------------------------ */

typedef struct {
    int64_t off, stride, trans, ld, group, inner;
} orc_matref;

static inline int64_t mat_base(const orc_matref *r, int64_t z) {
    int64_t g = r->group > 0 ? r->group : 1;
    return r->off + (z / g) * r->stride + (z % g) * r->inner;
}

/* out[z] (+)= epilogue(a[z] @ b[z]).  a[z] logically [m, k], b[z] [k, n].
 * ld == 0 means packed (the stored row length).  bias/mask/residual point at
 * their buffers already advanced by their offsets (or are NULL).  f16 != 0
 * rounds both operands to f16 before the product (the f16-in route).
 * Column sums of b[z] over k are added to out_buf[cs_off + z*cs_stride + j]
 * when has_cs; the sums use the f32 values (matmul.rs:75-77). */
void orc_gemm(const float *a_buf, const orc_matref *ar, const float *b_buf, const orc_matref *br,
              float *out_buf, const orc_matref *orf, int64_t batch, int64_t m, int64_t k, int64_t n,
              const float *bias, int64_t bias_stride, int32_t relu, const float *mask,
              const float *res, int32_t accumulate, int32_t has_cs, int64_t cs_off,
              int64_t cs_stride, int32_t f16) {
    int64_t lda = ar->ld ? ar->ld : (ar->trans ? m : k);
    int64_t ldb = br->ld ? br->ld : (br->trans ? k : n);
    int64_t ldo = orf->ld ? orf->ld : n;
    if (has_cs) {
        for (int64_t z = 0; z < batch; z++) {
            int64_t b0 = mat_base(br, z);
            for (int64_t j = 0; j < n; j++) {
                float s = 0.0f;
                for (int64_t p = 0; p < k; p++)
                    s += b_buf[b0 + (br->trans ? j * ldb + p : p * ldb + j)];
                out_buf[cs_off + z * cs_stride + j] += s;
            }
        }
    }
    for (int64_t z = 0; z < batch; z++) {
        int64_t a0 = mat_base(ar, z), b0 = mat_base(br, z);
        int64_t o0 = (z / (orf->group > 0 ? orf->group : 1)) * orf->stride +
                     (z % (orf->group > 0 ? orf->group : 1)) * orf->inner;
        /* Rows split over threads: each element's arithmetic is unchanged. */
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
        for (int64_t i = 0; i < m; i++) {
            for (int64_t j = 0; j < n; j++) {
                float s = 0.0f;
                for (int64_t p = 0; p < k; p++) {
                    float x = a_buf[a0 + (ar->trans ? p * lda + i : i * lda + p)];
                    float y = b_buf[b0 + (br->trans ? j * ldb + p : p * ldb + j)];
                    if (f16) {
                        x = orc_round_f16(x);
                        y = orc_round_f16(y);
                    }
                    s += x * y;
                }
                if (bias) s += bias[z * bias_stride + j];
                if (relu && s < 0.0f) s = 0.0f;
                int64_t idx = o0 + i * ldo + j;
                if (mask && mask[idx] <= 0.0f) s = 0.0f;
                if (res) s += res[idx];
                int64_t o = orf->off + idx;
                if (accumulate) s += out_buf[o];
                out_buf[o] = s;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Row softmax with causal mask, rows.rs:101-123 and k_softmax_fwd/bwd      */
/* rows.rs:295-357 (softmax1: tape.rs:425-435).                              */
/* ------------------------------------------------------------------------ */

/* y = softmax(scale*x) per row of [rows, n]; causal: row r sees columns
 * 0..=r%t, the rest are exactly 0; one: softmax1 (phantom logit 0, shift
 * max(rowmax, 0)).  Serial sums in f32. */
void orc_softmax(const float *x, float *y, int64_t rows, int64_t n, int64_t t, float scale,
                 int32_t causal, int32_t one) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * n;
        float *yr = y + r * n;
        int64_t limit = causal ? (r % t) + 1 : n;
        if (limit > n) limit = n;
        float mx = scale * xr[0];
        for (int64_t j = 1; j < limit; j++) {
            float v = scale * xr[j];
            if (v > mx) mx = v;
        }
        if (one && mx < 0.0f) mx = 0.0f;
        float s = 0.0f;
        for (int64_t j = 0; j < limit; j++) s += expf(scale * xr[j] - mx);
        if (one) s += expf(-mx);
        for (int64_t j = 0; j < n; j++) yr[j] = j < limit ? expf(scale * xr[j] - mx) / s : 0.0f;
    }
}

/* dx = scale * y * (dy - sum(dy * y)) per row (rows.rs:114-123). */
void orc_softmax_backward(const float *dy, const float *y, float *dx, int64_t rows, int64_t n,
                          float scale) {
    for (int64_t r = 0; r < rows; r++) {
        const float *a = dy + r * n, *b = y + r * n;
        float dot = 0.0f;
        for (int64_t j = 0; j < n; j++) dot += a[j] * b[j];
        for (int64_t j = 0; j < n; j++) dx[r * n + j] = scale * b[j] * (a[j] - dot);
    }
}

/* ------------------------------------------------------------------------ */
/* LayerNorm (nn.rs:306-321 `LayerNorm::forward_shared`, composed on the CPU */
/* tape; the device kernels rows.rs:65-99, 177-293).  Row r of x [rows, d]   */
/* uses gamma/beta at params[off + (r / rows_pm) * stride + j] and + d      */
/* (one parameter set per model of rows_pm rows).                            */
/* ------------------------------------------------------------------------ */

/* mean = (sum x) * (1/d); c = x - mean; var = (sum c^2) * (1/d) (biased);
 * std = sqrt(var + eps); y = (c / std) * gamma + beta; rstd = 1 / std.
 * Sums run in index order, every operation separately rounded, as the CPU
 * tape's sum_last_axis / scale / sub / mul / add / sqrt / div do. */
void orc_layer_norm(const float *x, int64_t rows, int64_t d, const float *params, int64_t off,
                    float eps, int64_t rows_pm, int64_t stride, float *y, float *mean, float *rstd) {
    const float inv_d = 1.0f / (float)d;
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * d;
        const float *gm = params + off + (r / rows_pm) * stride, *bt = gm + d;
        float s = 0.0f;
        for (int64_t j = 0; j < d; j++) s += xr[j];
        const float mu = s * inv_d;
        float sq = 0.0f;
        for (int64_t j = 0; j < d; j++) {
            const float c = xr[j] - mu;
            sq += c * c;
        }
        const float sd = sqrtf(sq * inv_d + eps);
        for (int64_t j = 0; j < d; j++) y[r * d + j] = ((xr[j] - mu) / sd) * gm[j] + bt[j];
        mean[r] = mu;
        rstd[r] = 1.0f / sd;
    }
}

/* The gradients of sum(dy * y): dx (+)= rstd (g - s1/d - xhat s2/d) with
 * g = dy gamma, xhat = (x - mean) rstd, s1 = sum g, s2 = sum g xhat
 * (rows.rs:221-267); grads[off + ...] += sum over the model's rows of dy xhat
 * (gamma) and dy (beta) (rows.rs:269-291), rows summed in index order. */
void orc_layer_norm_backward(const float *dy, const float *x, const float *mean, const float *rstd,
                             int64_t rows, int64_t d, const float *params, float *grads, int64_t off,
                             float *dx, int32_t accumulate, int64_t rows_pm, int64_t stride) {
    const float inv_d = 1.0f / (float)d;
    for (int64_t r = 0; r < rows; r++) {
        const float *gm = params + off + (r / rows_pm) * stride;
        const float mu = mean[r], rs = rstd[r];
        float s1 = 0.0f, s2 = 0.0f;
        for (int64_t j = 0; j < d; j++) {
            const float g = dy[r * d + j] * gm[j];
            s1 += g;
            s2 += g * ((x[r * d + j] - mu) * rs);
        }
        for (int64_t j = 0; j < d; j++) {
            const float g = dy[r * d + j] * gm[j];
            const float xh = (x[r * d + j] - mu) * rs;
            float v = rs * (g - s1 * inv_d - xh * (s2 * inv_d));
            dx[r * d + j] = accumulate ? dx[r * d + j] + v : v;
        }
    }
    const int64_t models = (rows + rows_pm - 1) / rows_pm;
    for (int64_t m = 0; m < models; m++) {
        float *gg = grads + off + m * stride, *gb = gg + d;
        for (int64_t j = 0; j < d; j++) {
            float pg = 0.0f, pb = 0.0f;
            for (int64_t r = m * rows_pm; r < (m + 1) * rows_pm && r < rows; r++) {
                pg += dy[r * d + j] * ((x[r * d + j] - mean[r]) * rstd[r]);
                pb += dy[r * d + j];
            }
            gg[j] += pg;
            gb[j] += pb;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Batched causal attention on the CPU tape path: batched_matmul_forward /   */
/* backward (tape.rs:73-112) over per-chunk NdArray::matmul with explicit    */
/* transposes, plus the causal softmax (nn.rs:396-407 mask, tape.rs:385-391).*/
/* Q, K, V, dO are [chunks*t, hd] stacked chunk-major; one: softmax1.        */
/* Outputs P [chunks*t, t], O [chunks*t, hd] and dQ, dK, dV.  scratch must   */
/* hold 4*t*t + 3*t*hd floats.  This is the CPU baseline of the attention    */
/* configuration.                                                            */
/* ------------------------------------------------------------------------ */
void orc_attention_fwd_bwd(const float *q, const float *kk, const float *v, const float *dout,
                           int64_t chunks, int64_t t, int64_t hd, float scale, int32_t one, float *p,
                           float *o, float *dq, float *dk, float *dv, float *scratch) {
    float *s = scratch;              /* [t, t] */
    float *kt = s + t * t;           /* [hd, t] */
    float *dp = kt + t * hd;         /* [t, t] */
    float *ds = dp + t * t;          /* [t, t] */
    float *tt = ds + t * t;          /* [t, t] transposes */
    float *th = tt + t * t;          /* [t, hd] or [hd, t] */
    float *th2 = th + t * hd;        /* [hd, t] */
    for (int64_t c = 0; c < chunks; c++) {
        const float *qc = q + c * t * hd, *kc = kk + c * t * hd, *vc = v + c * t * hd;
        const float *doc = dout + c * t * hd;
        float *pc = p + c * t * t, *oc = o + c * t * hd;
        /* S = Q K^T (batched_matmul_forward, transpose_b) */
        orc_transpose(kc, kt, t, hd);
        orc_matmul(qc, kt, s, t, hd, t);
        orc_softmax(s, pc, t, t, t, scale, 1, one);
        /* O = P V */
        orc_matmul(pc, vc, oc, t, t, hd);
        /* backward of O = P V: dP = dO V^T, dV = P^T dO */
        orc_transpose(vc, th2, t, hd);
        orc_matmul(doc, th2, dp, t, hd, t);
        orc_transpose(pc, tt, t, t);
        orc_matmul(tt, doc, dv + c * t * hd, t, t, hd);
        /* softmax backward */
        orc_softmax_backward(dp, pc, ds, t, t, scale);
        /* backward of S = Q K^T: dQ = dS K, dK = dS^T Q */
        orc_matmul(ds, kc, dq + c * t * hd, t, t, hd);
        orc_transpose(ds, tt, t, t);
        orc_matmul(tt, qc, dk + c * t * hd, t, t, hd);
        (void)th;
    }
}

/* ------------------------------------------------------------------------ */
/* 2-bit key store: quantiser tile_of, knn.rs:190-225 (bits = 2,             */
/* quant_step(2) = 0.9957, knn.rs:645-653).                                  */
/* ------------------------------------------------------------------------ */

/* Rust f32::round: half away from zero. */
static inline float round_half_away(float x) { return roundf(x); }

/* Row r of keys [n, d] -> codes (d/4 bytes, code i at byte i/4 bits 2(i%4),
 * low bits first), scale_r = max(0.9957 * sqrt(sum x^2 / d), 1e-30) with a
 * serial f32 sum; u = clamp(round(x / scale + 1.5), 0, 3).  norm_f16 (may be
 * NULL) gets the reference's stored norm, sum of f16((u - 1.5) * scale)^2. */
void orc_quantize_2bit(const float *keys, int64_t n, int64_t d, uint8_t *codes, float *scales,
                       float *norm_f16) {
    const float step = 0.9957f, half = 1.5f, top = 3.0f;
    int64_t kb = d / 4;
    for (int64_t r = 0; r < n; r++) {
        const float *k = keys + r * d;
        float ss = 0.0f;
        for (int64_t i = 0; i < d; i++) ss += k[i] * k[i];
        float scale = step * sqrtf(ss / (float)d);
        if (!(scale >= 1e-30f)) scale = 1e-30f;
        uint8_t *row = codes + r * kb;
        memset(row, 0, (size_t)kb);
        float nrm = 0.0f;
        for (int64_t i = 0; i < d; i++) {
            float u = round_half_away(k[i] / scale + half);
            if (u < 0.0f) u = 0.0f;
            if (u > top) u = top;
            int32_t c = (int32_t)u;
            row[i / 4] |= (uint8_t)((c & 3) << (2 * (i % 4)));
            float deq = orc_round_f16(((float)c - half) * scale);
            nrm += deq * deq;
        }
        scales[r] = scale;
        if (norm_f16) norm_f16[r] = nrm;
    }
}

/* ------------------------------------------------------------------------ */
/* Exact 2-bit scoring contract (the build's replacement for the reference's */
/* f16 cmma dots, ivf.rs:249-321, and distance, ivf.rs:235).                 */
/*                                                                            */
/* Query q (f32, d) -> power-of-two scale qs = 2^(E-14) where M = max|q_i| = */
/* m * 2^E, m in [0.5, 1) (qs = 1 when M == 0); Q_i = clamp(rint(q_i / qs),  */
/* -16384, 16383) (exact: qs is a power of two).  Key code u_i in 0..3 and   */
/* scale s decode to k_i = (u_i - 1.5) s = c_i s / 2 with c_i = 2u_i - 3.     */
/*   dot  = sum c_i Q_i                (exact int32)                          */
/*   c2   = sum c_i^2 = 256-ish..      (exact int32)                          */
/*   dist = ((s*s) * 0.25f) * (float)c2 - (s*qs) * (float)dot               */
/* each operation a separately rounded f32 op in that order (no FMA).        */
/* Ranking: ascending (dist, key index).  Reported distance:                 */
/*   max(qn + dist, 0) with qn = (float)(sum Q_i^2) * (qs*qs)                */
/* (the reference's finalisation (dd + |q|^2).max(0), ivf.rs:673-684).       */
/* ------------------------------------------------------------------------ */

typedef struct {
    float qs;     /* power-of-two query scale 2^qe */
    float qn;     /* |q^|^2 */
    int32_t sq;   /* sum Q_i */
    int32_t qe;   /* the scale's exponent */
} orc_qprep;

void orc_knn_prep_query(const float *q, int64_t d, int16_t *Q, orc_qprep *prep) {
    float mx = 0.0f;
    for (int64_t i = 0; i < d; i++) {
        float a = fabsf(q[i]);
        if (a > mx) mx = a;
    }
    int e = 14; /* scale 2^0 for a zero vector */
    if (mx > 0.0f) frexpf(mx, &e);
    const float qs = ldexpf(1.0f, e - 14);
    int64_t sq2 = 0;
    int32_t sq = 0;
    for (int64_t i = 0; i < d; i++) {
        /* q / 2^(e-14), exact (|result| < 2^14) even where 2^(e-14) is subnormal */
        float v = rintf(ldexpf(q[i], 14 - e));
        if (v > 16383.0f) v = 16383.0f;
        if (v < -16384.0f) v = -16384.0f;
        int32_t x = (int32_t)v;
        Q[i] = (int16_t)x;
        sq += x;
        sq2 += (int64_t)x * x;
    }
    prep->qs = qs;
    prep->qn = (float)sq2 * (qs * qs);
    prep->sq = sq;
    prep->qe = e - 14;
}

static inline float knn_dist(const uint8_t *code, float s, const int16_t *Q, float qs, int64_t d) {
    int32_t dot = 0, c2 = 0;
    for (int64_t i = 0; i < d; i++) {
        int32_t u = (code[i >> 2] >> (2 * (i & 3))) & 3;
        int32_t c = 2 * u - 3;
        dot += c * (int32_t)Q[i];
        c2 += c * c;
    }
    float a = (s * s) * 0.25f;
    float t1 = a * (float)c2;
    float t2 = s * qs;
    float t3 = t2 * (float)dot;
    return t1 - t3 + 0.0f; /* + 0.0f turns a -0 into +0 */
}

/* dist of every key of rows [r0, r1) for one prepared query. */
void orc_knn_dists(const uint8_t *codes, const float *scales, int64_t d, int64_t r0, int64_t r1,
                   const int16_t *Q, const orc_qprep *prep, float *out) {
    int64_t kb = d / 4;
    for (int64_t r = r0; r < r1; r++) out[r - r0] = knn_dist(codes + r * kb, scales[r], Q, prep->qs, d);
}

/* Monotone map of an f32 onto u32 (total order of the floats, -0 < +0). */
static inline uint32_t fkey(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    return (x & 0x80000000u) ? ~x : (x | 0x80000000u);
}

static inline void heap_sift_down(uint64_t *h, int64_t size, int64_t i) {
    uint64_t v = h[i];
    for (;;) {
        int64_t l = 2 * i + 1;
        if (l >= size) break;
        int64_t c = l;
        if (l + 1 < size && h[l + 1] > h[l]) c = l + 1;
        if (h[c] <= v) break;
        h[i] = h[c];
        i = c;
    }
    h[i] = v;
}

static int cmp_u64(const void *a, const void *b) {
    uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? -1 : x > y;
}

/* Top-k by (dist, key index) over the keys of each query's probed cells:
 * cells c occupy rows cell_start[c]..cell_start[c+1] of codes/scales;
 * probes [nq, nprobe] (a cell repeated within one query's probes is scanned
 * once).  Outputs out_idx [nq, k] (global row, -1 padding) and out_dist
 * [nq, k] (max(qn + dist, 0), +inf padding), ascending. */
void orc_knn_search(const uint8_t *codes, const float *scales, const int64_t *cell_start,
                    const float *queries, const int32_t *probes, int64_t nq, int64_t nprobe,
                    int64_t d, int64_t k, int64_t *out_idx, float *out_dist) {
    int64_t kb = d / 4;
#pragma omp parallel for schedule(dynamic) num_threads(g_threads) if (g_threads > 1)
    for (int64_t qi = 0; qi < nq; qi++) {
        int16_t *Q = (int16_t *)malloc(sizeof(int16_t) * (size_t)d);
        uint64_t *heap = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(k > 0 ? k : 1));
        orc_qprep prep;
        orc_knn_prep_query(queries + qi * d, d, Q, &prep);
        int64_t size = 0;
        for (int64_t pi = 0; pi < nprobe; pi++) {
            int32_t c = probes[qi * nprobe + pi];
            int dup = 0;
            for (int64_t pj = 0; pj < pi; pj++) dup |= probes[qi * nprobe + pj] == c;
            if (dup) continue;
            for (int64_t r = cell_start[c]; r < cell_start[c + 1]; r++) {
                float dist = knn_dist(codes + r * kb, scales[r], Q, prep.qs, d);
                uint64_t key = ((uint64_t)fkey(dist) << 32) | (uint64_t)(uint32_t)r;
                if (size < k) {
                    /* sift up */
                    int64_t i = size++;
                    while (i > 0) {
                        int64_t par = (i - 1) / 2;
                        if (heap[par] >= key) break;
                        heap[i] = heap[par];
                        i = par;
                    }
                    heap[i] = key;
                } else if (key < heap[0]) {
                    heap[0] = key;
                    heap_sift_down(heap, size, 0);
                }
            }
        }
        qsort(heap, (size_t)size, sizeof(uint64_t), cmp_u64);
        for (int64_t j = 0; j < k; j++) {
            if (j < size) {
                uint32_t fk = (uint32_t)(heap[j] >> 32);
                uint32_t bits = (fk & 0x80000000u) ? (fk & 0x7fffffffu) : ~fk;
                float dist;
                memcpy(&dist, &bits, 4);
                float v = prep.qn + dist;
                out_dist[qi * k + j] = v > 0.0f ? v : 0.0f;
                out_idx[qi * k + j] = (int64_t)(uint32_t)heap[j];
            } else {
                out_dist[qi * k + j] = INFINITY;
                out_idx[qi * k + j] = -1;
            }
        }
        free(heap);
        free(Q);
    }
}

/* The masked exact search (knn.rs:295-331 search_tagged / search_tail, the
 * key predicate of k_thresh / k_topk knn.rs:604-618): for query i, key g of
 * the store [0, n) takes part iff g < always or lo[i] <= g < hi[i]; top-k by
 * (dist, key index) over those keys, outputs as orc_knn_search. */
void orc_knn_search_masked(const uint8_t *codes, const float *scales, int64_t n, const float *queries,
                           const int64_t *lo, const int64_t *hi, int64_t always, int64_t nq, int64_t d,
                           int64_t k, int64_t *out_idx, float *out_dist) {
    int64_t kb = d / 4;
    int16_t *Q = (int16_t *)malloc(sizeof(int16_t) * (size_t)d);
    uint64_t *heap = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)k);
    for (int64_t qi = 0; qi < nq; qi++) {
        orc_qprep prep;
        orc_knn_prep_query(queries + qi * d, d, Q, &prep);
        int64_t size = 0;
        for (int64_t g = 0; g < n; g++) {
            if (!(g < always || (g >= lo[qi] && g < hi[qi]))) continue;
            float dist = knn_dist(codes + g * kb, scales[g], Q, prep.qs, d);
            uint64_t key = ((uint64_t)fkey(dist) << 32) | (uint64_t)(uint32_t)g;
            if (size < k) {
                int64_t i = size++;
                while (i > 0) {
                    int64_t par = (i - 1) / 2;
                    if (heap[par] >= key) break;
                    heap[i] = heap[par];
                    i = par;
                }
                heap[i] = key;
            } else if (key < heap[0]) {
                heap[0] = key;
                heap_sift_down(heap, size, 0);
            }
        }
        qsort(heap, (size_t)size, sizeof(uint64_t), cmp_u64);
        for (int64_t j = 0; j < k; j++) {
            if (j < size) {
                uint32_t fk = (uint32_t)(heap[j] >> 32);
                uint32_t bits = (fk & 0x80000000u) ? (fk & 0x7fffffffu) : ~fk;
                float dist;
                memcpy(&dist, &bits, 4);
                float v = prep.qn + dist;
                out_dist[qi * k + j] = v > 0.0f ? v : 0.0f;
                out_idx[qi * k + j] = (int64_t)(uint32_t)heap[j];
            } else {
                out_dist[qi * k + j] = INFINITY;
                out_idx[qi * k + j] = -1;
            }
        }
    }
    free(heap);
    free(Q);
}

/* The reference's own f16 scoring of one key, for fidelity checks: q and the
 * dequantised key both rounded to f16 (ivf.rs:470, k_dots_group ivf.rs:295-300),
 * dot summed in f32 in index order; returns |q^|^2 + norm - 2 q^.k^ with the
 * reference's stored norm (knn.rs:216). */
float orc_knn_ref_f16_dist(const uint8_t *code, float s, float norm_f16, const float *q, int64_t d) {
    float dot = 0.0f, qn = 0.0f;
    for (int64_t i = 0; i < d; i++) {
        int32_t u = (code[i >> 2] >> (2 * (i & 3))) & 3;
        float kv = orc_round_f16(((float)u - 1.5f) * s);
        float qv = orc_round_f16(q[i]);
        dot += qv * kv;
        qn += qv * qv;
    }
    return qn + norm_f16 - 2.0f * dot;
}

/* orc_knn_ref_f16_dist for every key of rows [r0, r1) against one query, into
 * out[r - r0] (same arithmetic; the four f16 key values of a key are rounded
 * once).  Fidelity measurement only: the reference's ranking next to the
 * exact integer contract's. */
void orc_knn_ref_f16_dists(const uint8_t *codes, const float *scales, const float *norm_f16, int64_t d,
                           int64_t r0, int64_t r1, const float *q, float *out) {
    float *qv = (float *)malloc(sizeof(float) * (size_t)d);
    float qn = 0.0f;
    for (int64_t i = 0; i < d; i++) {
        qv[i] = orc_round_f16(q[i]);
        qn += qv[i] * qv[i];
    }
    const int64_t kb = d / 4;
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int64_t r = r0; r < r1; r++) {
        const uint8_t *code = codes + r * kb;
        float lut[4];
        for (int u = 0; u < 4; u++) lut[u] = orc_round_f16(((float)u - 1.5f) * scales[r]);
        float dot = 0.0f;
        for (int64_t i = 0; i < d; i++) dot += qv[i] * lut[(code[i >> 2] >> (2 * (i & 3))) & 3];
        out[r - r0] = qn + norm_f16[r] - 2.0f * dot;
    }
    free(qv);
}

/* The reference's probe ranking (ivf.rs:62-67 `Cent::new`, ivf.rs:470-485 and
 * `k_probe` ivf.rs:131-161), for fidelity measurement: centroids and queries
 * rounded to f16, cnorm[c] = sum of the f16 centroid's squares in f32, dot =
 * the f16 products summed in f32 (index order here; the reference's matrix
 * cores may sum in another order), dd = cnorm - 2 dot, and the nprobe
 * smallest by insertion with strict <, so equal dd keep the lower cell. */
void orc_knn_ref_f16_probe(const float *cent, int64_t nlist, const float *queries, int64_t nq, int64_t d,
                           int64_t nprobe, int32_t *probes) {
    float *c16 = (float *)malloc(sizeof(float) * (size_t)(nlist * d));
    float *cnorm = (float *)malloc(sizeof(float) * (size_t)nlist);
    for (int64_t c = 0; c < nlist; c++) {
        float s = 0.0f;
        for (int64_t i = 0; i < d; i++) {
            const float x = orc_round_f16(cent[c * d + i]);
            c16[c * d + i] = x;
            s += x * x;
        }
        cnorm[c] = s;
    }
#pragma omp parallel for schedule(dynamic) num_threads(g_threads) if (g_threads > 1)
    for (int64_t qi = 0; qi < nq; qi++) {
        float *qv = (float *)malloc(sizeof(float) * (size_t)d);
        float *bd = (float *)malloc(sizeof(float) * (size_t)nprobe);
        int32_t *bi = (int32_t *)malloc(sizeof(int32_t) * (size_t)nprobe);
        for (int64_t i = 0; i < d; i++) qv[i] = orc_round_f16(queries[qi * d + i]);
        for (int64_t j = 0; j < nprobe; j++) {
            bd[j] = 3.0e38f;
            bi[j] = 0;
        }
        for (int64_t c = 0; c < nlist; c++) {
            float dot = 0.0f;
            for (int64_t i = 0; i < d; i++) dot += qv[i] * c16[c * d + i];
            const float dd = cnorm[c] - 2.0f * dot;
            if (!(dd < bd[nprobe - 1])) continue;
            int64_t pos = nprobe - 1;
            while (pos > 0 && bd[pos - 1] > dd) {
                bd[pos] = bd[pos - 1];
                bi[pos] = bi[pos - 1];
                pos--;
            }
            bd[pos] = dd;
            bi[pos] = (int32_t)c;
        }
        for (int64_t j = 0; j < nprobe; j++) probes[qi * nprobe + j] = bi[j];
        free(bi);
        free(bd);
        free(qv);
    }
    free(cnorm);
    free(c16);
}

/* ------------------------------------------------------------------------ */
/* Probe selection: each query's nprobe nearest IVF cells.                   */
/* ------------------------------------------------------------------------ */

/* The centroid side of probe selection (ivf.rs:62-69 `Cent::new`, with the
 * integer contract of the scan in place of f16 rounding): centroid c is
 * quantised exactly as a query (orc_knn_prep_query), C[c] = its int16 values,
 * cs = 2^cexp[c] its power-of-two scale, and cnorm[c] = |C cs|^2 =
 * ldexp(sum C^2, 2 cexp) in float64 (exact: sum C^2 < 2^37). */
void orc_knn_centroid_prep(const float *cent, int64_t nlist, int64_t d, int16_t *C, int32_t *cexp,
                           double *cnorm) {
    for (int64_t c = 0; c < nlist; c++) {
        orc_qprep p;
        orc_knn_prep_query(cent + c * d, d, C + c * d, &p);
        int64_t s2 = 0;
        for (int64_t i = 0; i < d; i++) s2 += (int64_t)C[c * d + i] * C[c * d + i];
        cexp[c] = p.qe;
        cnorm[c] = ldexp((double)s2, 2 * cexp[c]);
    }
}

/* ivf.rs:128-161 `k_probe` over the centroid dots of ivf.rs:473-484: for
 * each query (quantised as in the scan: Q, qs = 2^qe) and centroid c,
 *     dd = cnorm[c] - ldexp(dot, qe + cexp[c] + 1),   dot = sum Q_i C[c]_i
 * (dot exact in int64, dd one float64 subtraction), and the nprobe smallest
 * by (dd, c), nearest first, into probes [nq, nprobe]. */
void orc_knn_probe(const int16_t *C, const int32_t *cexp, const double *cnorm, int64_t nlist,
                   const float *queries, int64_t nq, int64_t d, int64_t nprobe, int32_t *probes) {
    int16_t *Q = (int16_t *)malloc(sizeof(int16_t) * (size_t)d);
    double *bd = (double *)malloc(sizeof(double) * (size_t)nprobe);
    int32_t *bi = (int32_t *)malloc(sizeof(int32_t) * (size_t)nprobe);
    for (int64_t qi = 0; qi < nq; qi++) {
        orc_qprep p;
        orc_knn_prep_query(queries + qi * d, d, Q, &p);
        const int qe = p.qe;
        int64_t size = 0;
        for (int64_t c = 0; c < nlist; c++) {
            int64_t dot = 0;
            const int16_t *cr = C + c * d;
            for (int64_t i = 0; i < d; i++) dot += (int64_t)Q[i] * cr[i];
            double dd = cnorm[c] - ldexp((double)dot, qe + cexp[c] + 1);
            if (size == nprobe && !(dd < bd[nprobe - 1])) continue;
            int64_t pos = size < nprobe ? size++ : nprobe - 1;
            while (pos > 0 && bd[pos - 1] > dd) {
                bd[pos] = bd[pos - 1];
                bi[pos] = bi[pos - 1];
                pos--;
            }
            bd[pos] = dd;
            bi[pos] = (int32_t)c;
        }
        for (int64_t j = 0; j < nprobe; j++) probes[qi * nprobe + j] = j < size ? bi[j] : -1;
    }
    free(bi);
    free(bd);
    free(Q);
}
