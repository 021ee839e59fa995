// GEMM for the three tape forms (C = A·B, dA = dC·Bᵀ, dB = Aᵀ·dC) on gfx950
// matrix cores, f32 and f16-in/f32-accumulate, batched, with head-view
// addressing, the reference's epilogue and deterministic split-k.
//
// Reference semantics: gpu_step/matmul.rs:26-299 (MatRef, Epilogue, matmul,
// matmul_f32, matmul_with, split-k and its ordered sum) and src/tensor.rs:241
// (NdArray::matmul).
//
// Design (gfx950 / CDNA4):
//  - One workgroup of 256 threads = 4 wave64s in a 2x2 grid computes a BM x BN
//    output tile; each wave owns (BM/2) x (BN/2) as 16x16 MFMA blocks.
//  - f16 route: v_mfma_f32_16x16x32_f16; f32 operands are read from HBM with
//    128-bit loads and rounded to f16 (round to nearest even) on the way into
//    LDS.  f32 route: v_mfma_f32_16x16x4_f32 on f32 LDS tiles.
//  - LDS holds both operands k-contiguous ([row][k], rows padded by 16 bytes
//    so the 128-bit fragment reads of 8 lanes hit distinct banks).  An operand
//    whose k is contiguous in memory (A not transposed, B transposed) is copied
//    as vectors; the others are loaded as 4x4 blocks and transposed in
//    registers.  k-stages of 64 (f16) / 32 (f32); two LDS buffers and two
//    register sets, so stage s+2 is in flight from global memory while stage s
//    feeds the MFMAs and stage s+1 is written to LDS; one barrier per stage.
//  - Workgroups are remapped so that each of the 8 XCDs works on a contiguous
//    run of tiles, which share operand panels in that XCD's L2.
//  - Fragment k-order: each lane reads its k-run as one 128-bit LDS read and
//    feeds it to the MFMA; A and B use the same k mapping, so the dot product
//    is over the right pairs whatever order the hardware sums them in.
//  - Split-k (shapes with too few output tiles, e.g. the weight gradients with
//    k = 4096): slices write [m, n] partials to the scratch arena, then one
//    launch sums them in slice order (deterministic), as the reference's
//    k_split_sum (matmul.rs:259-299).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#include "common.h"
#include "gemm_dma.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int THREADS = 256;

struct Operand {
    const float *p;  // buffer + element offset
    int64_t stride, group, inner, ld;
};

struct GemmArgs {
    Operand a, b;
    float *out;  // buffer + element offset (or the split-k partials)
    int64_t o_stride, o_group, o_inner, ldo;
    const float *bias;  // + bias_off
    int64_t bias_stride;
    const float *mask;  // + mask_off
    const float *res;   // + residual_off
    float *cs;          // column-sum destination (out buffer + col_sum_off, or partials)
    int64_t cs_stride;
    int32_t cs_direct, has_cs;
    int32_t m, n, k;
    int32_t splits, slice_k;
    int32_t relu, accumulate;
};

__device__ __forceinline__ int64_t mat_base(const Operand &o, int64_t z) {
    return (z / o.group) * o.stride + (z % o.group) * o.inner;
}

template <bool F16>
__device__ __forceinline__ void store4(void *dst, float x0, float x1, float x2, float x3) {
    if constexpr (F16) {
        half4 h = {(_Float16)x0, (_Float16)x1, (_Float16)x2, (_Float16)x3};
        *reinterpret_cast<half4 *>(dst) = h;
    } else {
        f32x4 v = {x0, x1, x2, x3};
        *reinterpret_cast<f32x4 *>(dst) = v;
    }
}

// Stages one operand's ROWS x BK tile (logical rows = m for A, n for B; k
// across) from global memory into registers, then into LDS as [row][k].
// KCONTIG: element (r, kk) at base[r*ld + kk]; else at base[kk*ld + r].
template <int ROWS, int BK, bool KCONTIG, bool FAST, bool F16>
struct Stager {
    static constexpr int LDS_K = BK + (F16 ? 8 : 4);
    // KCONTIG: 4-wide vectors along k.  Else 4x4 blocks (4 k x 4 rows).
    static constexpr int UNITS = KCONTIG ? ROWS * BK / 4 : ROWS * BK / 16;
    static constexpr int PER = (UNITS + THREADS - 1) / THREADS;
    static constexpr int VEC = KCONTIG ? 1 : 4;  // float4 per unit
    static constexpr int SLOTS = BK / 4;          // column-sum partials per row
    f32x4 r[PER][VEC];
    float cs[PER][KCONTIG ? 1 : 4];

    __device__ __forceinline__ void zero_cs() {
#pragma unroll
        for (int i = 0; i < PER; i++)
#pragma unroll
            for (int x = 0; x < (KCONTIG ? 1 : 4); x++) cs[i][x] = 0.f;
    }

    __device__ __forceinline__ void load(const float *__restrict__ base, int64_t ld, int row0,
                                         int row_lim, int k0, int k_lim, int tid) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int u = tid + THREADS * i;
            if (UNITS % THREADS != 0 && u >= UNITS) break;
            if constexpr (KCONTIG) {
                const int rr = u / (BK / 4), kq = (u % (BK / 4)) * 4;
                const float *src = base + (int64_t)(row0 + rr) * ld + (k0 + kq);
                if constexpr (FAST) {
                    r[i][0] = *reinterpret_cast<const f32x4 *>(src);
                } else {
                    const bool rok = row0 + rr < row_lim;
#pragma unroll
                    for (int e = 0; e < 4; e++) r[i][0][e] = (rok && k0 + kq + e < k_lim) ? src[e] : 0.f;
                }
            } else {
                const int rq = (u % (ROWS / 4)) * 4, kq = (u / (ROWS / 4)) * 4;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float *src = base + (int64_t)(k0 + kq + e) * ld + (row0 + rq);
                    if constexpr (FAST) {
                        r[i][e] = *reinterpret_cast<const f32x4 *>(src);
                    } else {
                        const bool kok = k0 + kq + e < k_lim;
#pragma unroll
                        for (int x = 0; x < 4; x++) r[i][e][x] = (kok && row0 + rq + x < row_lim) ? src[x] : 0.f;
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void add_cs() {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            if constexpr (KCONTIG) {
                cs[i][0] += ((r[i][0][0] + r[i][0][1]) + r[i][0][2]) + r[i][0][3];
            } else {
#pragma unroll
                for (int x = 0; x < 4; x++) cs[i][x] += ((r[i][0][x] + r[i][1][x]) + r[i][2][x]) + r[i][3][x];
            }
        }
    }

    template <typename T>
    __device__ __forceinline__ void store(T *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int u = tid + THREADS * i;
            if (UNITS % THREADS != 0 && u >= UNITS) break;
            if constexpr (KCONTIG) {
                const int rr = u / (BK / 4), kq = (u % (BK / 4)) * 4;
                store4<F16>(lds + rr * LDS_K + kq, r[i][0][0], r[i][0][1], r[i][0][2], r[i][0][3]);
            } else {
                const int rq = (u % (ROWS / 4)) * 4, kq = (u / (ROWS / 4)) * 4;
#pragma unroll
                for (int x = 0; x < 4; x++)
                    store4<F16>(lds + (rq + x) * LDS_K + kq, r[i][0][x], r[i][1][x], r[i][2][x], r[i][3][x]);
            }
        }
    }

    __device__ __forceinline__ void merge_cs(const Stager &o) {
#pragma unroll
        for (int i = 0; i < PER; i++)
#pragma unroll
            for (int x = 0; x < (KCONTIG ? 1 : 4); x++) cs[i][x] += o.cs[i][x];
    }

    // Writes this thread's column-sum partials to red[col * SLOTS + slot].
    __device__ __forceinline__ void put_cs(float *red, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int u = tid + THREADS * i;
            if (UNITS % THREADS != 0 && u >= UNITS) break;
            if constexpr (KCONTIG) {
                red[(u / (BK / 4)) * SLOTS + u % (BK / 4)] = cs[i][0];
            } else {
                const int rq = (u % (ROWS / 4)) * 4, slot = u / (ROWS / 4);
#pragma unroll
                for (int x = 0; x < 4; x++) red[(rq + x) * SLOTS + slot] = cs[i][x];
            }
        }
    }
};

template <int BM, int BN, int BK, bool TA, bool TB, bool F16, bool FAST>
__global__ __launch_bounds__(THREADS) void k_gemm(GemmArgs g) {
    using T = typename std::conditional<F16, _Float16, float>::type;
    using SA = Stager<BM, BK, !TA, FAST, F16>;
    using SB = Stager<BN, BK, TB, FAST, F16>;
    constexpr int LDS_K = SA::LDS_K;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 16, FN = WN / 16;
    static_assert(BK % (F16 ? 32 : 16) == 0, "k stage");
    __shared__ __attribute__((aligned(16))) T As[2][BM * LDS_K];
    __shared__ __attribute__((aligned(16))) T Bs[2][BN * LDS_K];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // Workgroups are dealt to the 8 XCDs round-robin by linear id; remap so
    // each XCD gets a contiguous run of tiles (x fastest), which share A rows
    // (and k-slices) in that XCD's L2.
    int64_t lin = blockIdx.x + (int64_t)gridDim.x * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
    const int64_t total = (int64_t)gridDim.x * gridDim.y * gridDim.z;
    if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
    const int bx = (int)(lin % gridDim.x);
    const int by = (int)((lin / gridDim.x) % gridDim.y);
    const int64_t z = lin / ((int64_t)gridDim.x * gridDim.y);
    const int64_t zb = z / g.splits;
    const int slice = (int)(z % g.splits);
    const int row0 = by * BM, col0 = bx * BN;
    const int kbeg = slice * g.slice_k;
    const int kend = min(g.k, kbeg + g.slice_k);
    const int nst = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    const float *abase = g.a.p + mat_base(g.a, zb);
    const float *bbase = g.b.p + mat_base(g.b, zb);
    const bool do_cs = g.has_cs && by == 0;

    // Two register sets: stage st+2 is fetched into the set stage st came
    // from while stage st is multiplied out of LDS, so two stages of global
    // loads are in flight behind every barrier.
    SA sa[2];
    SB sb[2];
    sb[0].zero_cs();
    sb[1].zero_cs();
    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (nst > 0) {
        sa[0].load(abase, g.a.ld, row0, g.m, kbeg, kend, tid);
        sb[0].load(bbase, g.b.ld, col0, g.n, kbeg, kend, tid);
    }
    if (nst > 1) {
        sa[1].load(abase, g.a.ld, row0, g.m, kbeg + BK, kend, tid);
        sb[1].load(bbase, g.b.ld, col0, g.n, kbeg + BK, kend, tid);
    }
    if (nst > 0) {
        if (do_cs) sb[0].add_cs();
        sa[0].store(As[0], tid);
        sb[0].store(Bs[0], tid);
    }
    __syncthreads();

    auto body = [&](auto pc, int st) {
        constexpr int P = decltype(pc)::value;
        if (st + 2 < nst) {
            const int k0 = kbeg + (st + 2) * BK;
            sa[P].load(abase, g.a.ld, row0, g.m, k0, kend, tid);
            sb[P].load(bbase, g.b.ld, col0, g.n, k0, kend, tid);
        }
        const T *as = As[P] + (wm * WM + (lane & 15)) * LDS_K;
        const T *bs = Bs[P] + (wn * WN + (lane & 15)) * LDS_K;
        if constexpr (F16) {
#pragma unroll
            for (int ks = 0; ks < BK / 32; ks++) {
                half8 af[FM], bf[FN];
                const int ko = ks * 32 + 8 * (lane >> 4);
#pragma unroll
                for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const half8 *>(as + i * 16 * LDS_K + ko);
#pragma unroll
                for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const half8 *>(bs + j * 16 * LDS_K + ko);
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int kc = 0; kc < BK / 16; kc++) {
                f32x4 af[FM], bf[FN];
                const int ko = kc * 16 + 4 * (lane >> 4);
#pragma unroll
                for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const f32x4 *>(as + i * 16 * LDS_K + ko);
#pragma unroll
                for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const f32x4 *>(bs + j * 16 * LDS_K + ko);
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < FM; i++)
#pragma unroll
                        for (int j = 0; j < FN; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
            }
        }
        if (st + 1 < nst) {
            if (do_cs) sb[P ^ 1].add_cs();
            sa[P ^ 1].store(As[P ^ 1], tid);
            sb[P ^ 1].store(Bs[P ^ 1], tid);
        }
        __syncthreads();
    };
    for (int st = 0; st < nst; st += 2) {
        body(std::integral_constant<int, 0>(), st);
        if (st + 1 < nst) body(std::integral_constant<int, 1>(), st + 1);
    }

    // Column sums of this slice of B (tile row 0 only), reduced in slot order.
    if (do_cs) {
        float *red = reinterpret_cast<float *>(As[0]);  // BN * SLOTS floats fit in As
        static_assert(BN * SB::SLOTS * 4 <= BM * LDS_K * (int)sizeof(T), "column-sum buffer");
        sb[0].merge_cs(sb[1]);
        sb[0].put_cs(red, tid);
        __syncthreads();
        if (tid < BN && col0 + tid < g.n) {
            float tot = 0.f;
#pragma unroll
            for (int s = 0; s < SB::SLOTS; s++) tot += red[tid * SB::SLOTS + s];
            float *dst = g.cs + (g.cs_direct ? zb : z) * g.cs_stride + col0 + tid;
            if (g.cs_direct)
                *dst += tot;
            else
                *dst = tot;
        }
    }

    // Epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each block.
    const int64_t o0 = (z / g.o_group) * g.o_stride + (z % g.o_group) * g.o_inner;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = col0 + wn * WN + j * 16 + (lane & 15);
            if (!FAST && col >= g.n) continue;
            const float bv = g.bias ? g.bias[zb * g.bias_stride + col] : 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = row0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                if (!FAST && row >= g.m) continue;
                float v = acc[i][j][r];
                const int64_t idx = o0 + (int64_t)row * g.ldo + col;
                if (g.bias) v += bv;
                if (g.relu && v < 0.f) v = 0.f;
                if (g.mask && g.mask[idx] <= 0.f) v = 0.f;
                if (g.res) v += g.res[idx];
                if (g.accumulate) v += g.out[idx];
                g.out[idx] = v;
            }
        }
    }
}

// out[b] (+)= sum over s (ascending) of partial[b*splits + s]; then the
// column-sum partials into their destination (always +=).
__global__ __launch_bounds__(256) void k_split_sum(const float *__restrict__ partial, float *out,
                                                   int64_t len, int32_t splits, int64_t o_stride,
                                                   int64_t batch, int32_t accumulate, const float *cs_part,
                                                   float *cs_dst, int64_t cs_stride, int64_t n) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < batch * len) {
        const int64_t b = e / len, i = e % len;
        float v = 0.f;
        for (int s = 0; s < splits; s++) v += partial[(b * splits + s) * len + i];
        float *o = out + b * o_stride + i;
        if (accumulate) v += *o;
        *o = v;
    } else if (cs_part) {
        const int64_t c = e - batch * len;
        if (c < batch * n) {
            const int64_t b = c / n, j = c % n;
            float v = 0.f;
            for (int s = 0; s < splits; s++) v += cs_part[(b * splits + s) * n + j];
            cs_dst[b * cs_stride + j] += v;
        }
    }
}

using KernelFn = void (*)(GemmArgs);

template <int BM, int BN, int BK, bool F16>
KernelFn pick_kernel(bool ta, bool tb, bool fast) {
#define ST_K(TA, TB, FA) &k_gemm<BM, BN, BK, TA, TB, F16, FA>
    if (fast) {
        if (!ta && !tb) return ST_K(false, false, true);
        if (!ta && tb) return ST_K(false, true, true);
        if (ta && !tb) return ST_K(true, false, true);
        return ST_K(true, true, true);
    }
    if (!ta && !tb) return ST_K(false, false, false);
    if (!ta && tb) return ST_K(false, true, false);
    if (ta && !tb) return ST_K(true, false, false);
    return ST_K(true, true, false);
#undef ST_K
}

struct TileCfg {
    int bm, bn;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Output tile for a problem: the largest of 128x128, 128x64, 64x64 that gives
// at least one wave of workgroups (256 CUs), else 64x64.
TileCfg choose_tile(int64_t batch, int64_t m, int64_t n) {
    const int64_t cus = 256;
    if (batch * cdiv(m, 128) * cdiv(n, 128) >= cus) return {128, 128};
    if (batch * cdiv(m, 128) * cdiv(n, 64) >= cus) return {128, 64};
    return {64, 64};
}

bool aligned4(const float *p, int64_t off, int64_t stride, int64_t inner, int64_t ld) {
    return ((reinterpret_cast<uintptr_t>(p + off) & 15) == 0) && stride % 4 == 0 && inner % 4 == 0 && ld % 4 == 0;
}

st_status check_ref(const st_matref *r, const char *what) {
    if (!r) return st::fail(ST_ERR_INVALID, "%s is NULL", what);
    if (!r->p) return st::fail(ST_ERR_INVALID, "%s.p is NULL", what);
    if (r->off < 0 || r->stride < 0 || r->ld < 0 || r->group < 0 || r->inner < 0)
        return st::fail(ST_ERR_INVALID, "%s has a negative offset, stride, ld, group or inner", what);
    return ST_OK;
}

// The reference's argument checks for one call (its assert!s).
st_status check_call(const st_matref *a, const st_matref *b, const st_matref *out, int64_t batch, int64_t m,
                     int64_t k, int64_t n) {
    st_status s;
    if ((s = check_ref(a, "a")) || (s = check_ref(b, "b")) || (s = check_ref(out, "out"))) return s;
    if (out->trans) return st::fail(ST_ERR_INVALID, "out is stored row-major");
    if (batch < 0 || m < 0 || k < 0 || n < 0) return st::fail(ST_ERR_INVALID, "negative batch or shape");
    if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
        return st::fail(ST_ERR_INVALID, "matrix dimension too large");
    return ST_OK;
}

// The reference's f16 eligibility (matmul.rs:108-112, 524-534): k % 32, m % 64
// and n % 64 (or n % 32 for its 64x32 tile), and not column sums of a
// transposed b.
bool f16_route(bool use_f16, const st_epilogue &epi, const st_matref *b, int64_t m, int64_t k, int64_t n) {
    return use_f16 && !(epi.has_col_sum && b->trans) && k > 0 && k % 32 == 0 && m % 64 == 0 && n % 32 == 0;
}

// One call as the LDS-DMA kernels take it: element offsets folded into the
// pointers, group 0 read as 1, packed leading dimensions made explicit.
st::DmaGemm make_dma(const st_matref *a, const st_matref *b, const st_matref *out, int64_t batch, int64_t m,
                     int64_t k, int64_t n, const st_epilogue &epi, bool f16) {
    st::DmaGemm d;
    std::memset(&d, 0, sizeof d);
    d.a = a->p + a->off;
    d.a_stride = a->stride;
    d.a_group = a->group > 0 ? a->group : 1;
    d.a_inner = a->inner;
    d.lda = a->ld ? a->ld : (a->trans ? m : k);
    d.ta = a->trans != 0;
    d.b = b->p + b->off;
    d.b_stride = b->stride;
    d.b_group = b->group > 0 ? b->group : 1;
    d.b_inner = b->inner;
    d.ldb = b->ld ? b->ld : (b->trans ? k : n);
    d.tb = b->trans != 0;
    d.out = out->p + out->off;
    d.o_stride = out->stride;
    d.o_group = out->group > 0 ? out->group : 1;
    d.o_inner = out->inner;
    d.ldo = out->ld ? out->ld : n;
    d.bias = epi.bias ? epi.bias + epi.bias_off : nullptr;
    d.bias_stride = epi.bias_stride;
    d.mask = epi.mask ? epi.mask + epi.mask_off : nullptr;
    d.res = epi.residual ? epi.residual + epi.residual_off : nullptr;
    d.cs = out->p + epi.col_sum_off;
    d.cs_stride = epi.col_sum_stride;
    d.has_cs = epi.has_col_sum;
    d.relu = epi.relu;
    d.accumulate = epi.accumulate;
    d.f16 = f16;
    d.batch = batch;
    d.m = m;
    d.k = k;
    d.n = n;
    return d;
}

// Split-k of the any-shape kernel, as the reference allows it
// (matmul.rs:117-123): no epilogue but +=, packed out, and only when the
// output tiles alone leave CUs idle.  Enough slices to give every CU a
// workgroup, each keeping at least 4 k-stages.
void kgemm_splits(const TileCfg &tc, int BK, const st_epilogue &epi, const st_matref *out, int64_t batch, int64_t m,
                  int64_t k, int64_t n, int64_t &splits, int64_t &slice_k) {
    const int64_t tiles = batch * cdiv(m, tc.bm) * cdiv(n, tc.bn);
    const int64_t og = out->group > 0 ? out->group : 1;
    const bool epi_free = !epi.bias && !epi.relu && !epi.mask && !epi.residual;
    const bool packed_out = (out->ld == 0 || out->ld == n) && og == 1;
    splits = 1;
    const int64_t cus = 256;
    if (epi_free && packed_out && tiles < cus)
        splits = std::max<int64_t>(1, std::min<int64_t>(cdiv(cus, tiles), k / (4 * BK)));
    slice_k = cdiv(cdiv(k, splits), BK) * BK;
    if (slice_k == 0) slice_k = BK;
    splits = std::max<int64_t>(1, cdiv(k, slice_k));
}

// Bytes of split-k scratch gemm_impl would request for these arguments (0
// when it would request none or refuse them).
size_t gemm_impl_scratch(const st_matref *a, const st_matref *b, const st_matref *out, int64_t batch, int64_t m,
                         int64_t k, int64_t n, const st_epilogue &epi, bool use_f16) {
    if (!a || !b || !out || !a->p || !b->p || !out->p || out->trans || batch <= 0 || m <= 0 || n <= 0 || k <= 0)
        return 0;
    const bool f16 = f16_route(use_f16, epi, b, m, k, n);
    const st::DmaGemm d = make_dma(a, b, out, batch, m, k, n, epi, f16);
    size_t dma = 0;
    if ((dma = st::gemm_dma_scratch(d)) || st::gemm_dma_takes(d)) return dma;
    const TileCfg tc = choose_tile(batch, m, n);
    int64_t splits = 1, slice_k = 0;
    kgemm_splits(tc, f16 ? 64 : 32, epi, out, batch, m, k, n, splits, slice_k);
    if (splits <= 1) return 0;
    return sizeof(float) * (size_t)(batch * splits * m * n + (epi.has_col_sum ? batch * splits * n : 0));
}

st_status gemm_impl(const st_matref *a, const st_matref *b, const st_matref *out, int64_t batch, int64_t m,
                    int64_t k, int64_t n, const st_epilogue *epi_in, bool use_f16, hipStream_t stream) {
    st::clear_error();
    st_status s;
    if ((s = check_call(a, b, out, batch, m, k, n))) return s;
    st_epilogue epi;
    std::memset(&epi, 0, sizeof epi);
    if (epi_in) epi = *epi_in;
    if (batch == 0 || m == 0 || n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;

    const bool f16 = f16_route(use_f16, epi, b, m, k, n);
    const int64_t ag = a->group > 0 ? a->group : 1, bg = b->group > 0 ? b->group : 1;
    const int64_t og = out->group > 0 ? out->group : 1;
    const int64_t lda = a->ld ? a->ld : (a->trans ? m : k);
    const int64_t ldb = b->ld ? b->ld : (b->trans ? k : n);
    const int64_t ldo = out->ld ? out->ld : n;

    // Tile-divisible, 16-byte aligned problems run on the LDS-DMA kernel.
    {
        st_status ds = ST_OK;
        if (st::gemm_dma(make_dma(a, b, out, batch, m, k, n, epi, f16), stream, &ds)) return ds;
    }

    TileCfg tc = choose_tile(batch, m, n);
    const int BK = f16 ? 64 : 32;
    int64_t splits = 1, slice_k = 0;
    kgemm_splits(tc, BK, epi, out, batch, m, k, n, splits, slice_k);
    if (batch * splits > 65535) return st::fail(ST_ERR_INVALID, "batch %lld too large for one launch", (long long)batch);
    if (cdiv(m, tc.bm) > 65535) return st::fail(ST_ERR_INVALID, "m = %lld too large for one launch", (long long)m);

    GemmArgs g;
    std::memset(&g, 0, sizeof g);
    g.a = {a->p + a->off, a->stride, ag, a->inner, lda};
    g.b = {b->p + b->off, b->stride, bg, b->inner, ldb};
    g.m = (int32_t)m;
    g.n = (int32_t)n;
    g.k = (int32_t)k;
    g.splits = (int32_t)splits;
    g.slice_k = (int32_t)slice_k;

    float *partial = nullptr;
    if (splits > 1) {
        const size_t base = (size_t)(batch * splits * m * n);
        const size_t extra = epi.has_col_sum ? (size_t)(batch * splits * n) : 0;
        partial = static_cast<float *>(st::scratch(st::SCRATCH_SPLITK, (base + extra) * sizeof(float), stream));
        if (!partial) return st::scratch_status();
        g.out = partial;
        g.o_stride = m * n;
        g.o_group = 1;
        g.o_inner = 0;
        g.ldo = n;
        g.has_cs = epi.has_col_sum;
        g.cs = partial + base;
        g.cs_stride = n;
        g.cs_direct = 0;
    } else {
        g.out = out->p + out->off;
        g.o_stride = out->stride;
        g.o_group = og;
        g.o_inner = out->inner;
        g.ldo = ldo;
        g.bias = epi.bias ? epi.bias + epi.bias_off : nullptr;
        g.bias_stride = epi.bias_stride;
        g.mask = epi.mask ? epi.mask + epi.mask_off : nullptr;
        g.res = epi.residual ? epi.residual + epi.residual_off : nullptr;
        g.relu = epi.relu;
        g.accumulate = epi.accumulate;
        g.has_cs = epi.has_col_sum;
        g.cs = out->p + epi.col_sum_off;
        g.cs_stride = epi.col_sum_stride;
        g.cs_direct = 1;
    }

    const bool fast = m % tc.bm == 0 && n % tc.bn == 0 && k % BK == 0 && slice_k % BK == 0 &&
                      aligned4(a->p, a->off, a->stride, a->inner, lda) && aligned4(b->p, b->off, b->stride, b->inner, ldb);
    KernelFn fn;
    if (f16) {
        if (tc.bm == 128 && tc.bn == 128) fn = pick_kernel<128, 128, 64, true>(a->trans, b->trans, fast);
        else if (tc.bm == 128) fn = pick_kernel<128, 64, 64, true>(a->trans, b->trans, fast);
        else fn = pick_kernel<64, 64, 64, true>(a->trans, b->trans, fast);
    } else {
        if (tc.bm == 128 && tc.bn == 128) fn = pick_kernel<128, 128, 32, false>(a->trans, b->trans, fast);
        else if (tc.bm == 128) fn = pick_kernel<128, 64, 32, false>(a->trans, b->trans, fast);
        else fn = pick_kernel<64, 64, 32, false>(a->trans, b->trans, fast);
    }
    dim3 grid((unsigned)cdiv(n, tc.bn), (unsigned)cdiv(m, tc.bm), (unsigned)(batch * splits));
    hipLaunchKernelGGL(fn, grid, dim3(THREADS), 0, stream, g);
    ST_LAUNCH_CHECK();

    if (splits > 1) {
        const int64_t len = m * n;
        const int64_t total = batch * (len + (epi.has_col_sum ? n : 0));
        hipLaunchKernelGGL(k_split_sum, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, stream, partial,
                           out->p + out->off, len, (int32_t)splits, out->stride, batch, (int32_t)epi.accumulate,
                           epi.has_col_sum ? partial + batch * splits * len : nullptr, out->p + epi.col_sum_off,
                           epi.col_sum_stride, n);
        ST_LAUNCH_CHECK();
    }
    return ST_OK;
}

}  // namespace

extern "C" int32_t st_f16_enabled(void) {
    static const int32_t on = [] {
        const char *v = std::getenv("TRAIN_F16");
        return (v && std::strcmp(v, "0") == 0) ? 0 : 1;
    }();
    return on;
}

extern "C" st_status st_matmul(const st_matref *a, const st_matref *b, const st_matref *out, int64_t batch,
                               int64_t m, int64_t k, int64_t n, const st_epilogue *epi, st_stream stream) {
    return gemm_impl(a, b, out, batch, m, k, n, epi, st_f16_enabled() != 0, st::stream_of(stream));
}

extern "C" st_status st_matmul_f32(const st_matref *a, const st_matref *b, const st_matref *out, int64_t batch,
                                   int64_t m, int64_t k, int64_t n, const st_epilogue *epi, st_stream stream) {
    return gemm_impl(a, b, out, batch, m, k, n, epi, false, st::stream_of(stream));
}

extern "C" st_status st_matmul_with(const st_matref *a, const st_matref *b, const st_matref *out,
                                    int64_t batch, int64_t m, int64_t k, int64_t n, const st_epilogue *epi,
                                    int32_t use_f16, st_stream stream) {
    return gemm_impl(a, b, out, batch, m, k, n, epi, use_f16 != 0, st::stream_of(stream));
}

extern "C" st_status st_matmul_grouped(const st_gemm *gemms, int64_t count, st_stream stream) {
    st::clear_error();
    if (count < 0 || (count > 0 && !gemms)) return st::fail(ST_ERR_INVALID, "grouped GEMM: bad count or NULL array");
    for (int64_t i = 0; i < count; i++) {
        const st_gemm &g = gemms[i];
        const st_status s = check_call(&g.a, &g.b, &g.out, g.batch, g.m, g.k, g.n);
        if (s) {
            const std::string msg = st_last_error();
            return st::fail(s, "GEMM %lld of the group: %s", (long long)i, msg.c_str());
        }
    }
    if (count == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const hipStream_t s = st::stream_of(stream);
    std::vector<st::DmaGemm> elig[2];  // by route (f32, f16)
    std::vector<int64_t> rest;
    for (int64_t i = 0; i < count; i++) {
        const st_gemm &g = gemms[i];
        if (g.batch == 0 || g.m == 0 || g.n == 0) continue;
        const bool f16 = f16_route(g.use_f16 != 0, g.epi, &g.b, g.m, g.k, g.n);
        const st::DmaGemm d = make_dma(&g.a, &g.b, &g.out, g.batch, g.m, g.k, g.n, g.epi, f16);
        if (st::group_eligible(d))
            elig[f16 ? 1 : 0].push_back(d);
        else
            rest.push_back(i);
    }
    // 256-row tiles only when the route's GEMMs give every CU at least one of
    // them; a small group (a single Linear backward) keeps 128-row tiles.
    std::vector<st::DmaGemm> grp[4];  // route + 2 * (256-row tiles)
    for (int f = 0; f < 2; f++) {
        int64_t tall_tiles = 0;
        for (const st::DmaGemm &d : elig[f])
            if (st::group_tall(d)) tall_tiles += d.batch * (d.m / 256) * (d.n / 128);
        const bool use_tall = tall_tiles >= 256;
        for (const st::DmaGemm &d : elig[f]) grp[f + 2 * (use_tall && st::group_tall(d))].push_back(d);
    }
    // All or nothing: the launches below share the split-k scratch one after
    // another, so the largest need among them is requested before the first
    // launch.  A refusal (a fixed scratch too small, an arena that cannot grow
    // under graph capture or out of memory) then leaves every output as it
    // was; every later request fits what is already there.
    size_t need = 0;
    for (int f = 0; f < 4; f++)
        for (size_t c = 0; c < grp[f].size(); c += st::GROUP_MAX) {
            const int cnt = (int)std::min<size_t>(st::GROUP_MAX, grp[f].size() - c);
            need = std::max(need, st::gemm_group_scratch(grp[f].data() + c, cnt, (f & 1) != 0, (f & 2) != 0));
        }
    for (const int64_t i : rest) {
        const st_gemm &g = gemms[i];
        need = std::max(need, gemm_impl_scratch(&g.a, &g.b, &g.out, g.batch, g.m, g.k, g.n, g.epi, g.use_f16 != 0));
    }
    if (need && !st::scratch(st::SCRATCH_SPLITK, need, s)) return st::scratch_status();
    for (int f = 0; f < 4; f++)
        for (size_t c = 0; c < grp[f].size(); c += st::GROUP_MAX) {
            const int cnt = (int)std::min<size_t>(st::GROUP_MAX, grp[f].size() - c);
            const st_status r = st::gemm_group(grp[f].data() + c, cnt, (f & 1) != 0, (f & 2) != 0, s);
            if (r) return r;
        }
    for (const int64_t i : rest) {
        const st_gemm &g = gemms[i];
        const st_status r = gemm_impl(&g.a, &g.b, &g.out, g.batch, g.m, g.k, g.n, &g.epi, g.use_f16 != 0, s);
        if (r) return r;
    }
    return ST_OK;
}

extern "C" st_status st_ndarray_matmul(const float *a, const float *b, float *out, int64_t m, int64_t k,
                                       int64_t n) {
    st::clear_error();
    if (!a || !b || !out) return st::fail(ST_ERR_INVALID, "NULL host buffer");
    if (m < 0 || k < 0 || n < 0) return st::fail(ST_ERR_INVALID, "negative shape");
    if (m == 0 || n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    hipStream_t s;
    ST_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    // Split-k partials in buffers of this call's own (freed when it returns):
    // concurrent calls never share the library's arena.
    st::ScratchScope private_scratch;
    float *da = nullptr, *db = nullptr, *dc = nullptr;
    st_status rc = ST_OK;
    const size_t ba = sizeof(float) * (size_t)(m * k), bb = sizeof(float) * (size_t)(k * n),
                 bc = sizeof(float) * (size_t)(m * n);
    auto cleanup = [&] {
        (void)hipStreamSynchronize(s);
        if (da) (void)hipFree(da);
        if (db) (void)hipFree(db);
        if (dc) (void)hipFree(dc);
        (void)hipStreamDestroy(s);
    };
    if (hipMalloc(&da, ba ? ba : 4) != hipSuccess || hipMalloc(&db, bb ? bb : 4) != hipSuccess ||
        hipMalloc(&dc, bc) != hipSuccess) {
        (void)hipGetLastError();
        cleanup();
        return st::fail(ST_ERR_OOM, "device allocation for NdArray::matmul failed");
    }
    if ((ba && hipMemcpyAsync(da, a, ba, hipMemcpyHostToDevice, s) != hipSuccess) ||
        (bb && hipMemcpyAsync(db, b, bb, hipMemcpyHostToDevice, s) != hipSuccess)) {
        cleanup();
        return st::fail(ST_ERR_HIP, "host to device copy failed");
    }
    st_matref ra{da, 0, 0, 0, 0, 0, 1, 0}, rb{db, 0, 0, 0, 0, 0, 1, 0}, rc_{dc, 0, 0, 0, 0, 0, 1, 0};
    if (k == 0) {
        if (hipMemsetAsync(dc, 0, bc, s) != hipSuccess) rc = st::fail(ST_ERR_HIP, "hipMemsetAsync failed");
    } else {
        rc = gemm_impl(&ra, &rb, &rc_, 1, m, k, n, nullptr, false, s);
    }
    if (rc == ST_OK && hipMemcpyAsync(out, dc, bc, hipMemcpyDeviceToHost, s) != hipSuccess)
        rc = st::fail(ST_ERR_HIP, "device to host copy failed");
    if (rc == ST_OK && hipStreamSynchronize(s) != hipSuccess) rc = st::fail(ST_ERR_HIP, "stream synchronize failed");
    cleanup();
    return rc;
}
