// Fused causal attention on gfx950: forward and backward without materialising
// the scores or probabilities.
//
// Reference semantics: tape.rs:73-112 (batched attention forward/backward as
// per-chunk products), gpu_step/tape.rs:196-212, 349-372 (the device tape's
// batched products over head views of the fused QKV buffer), rows.rs:101-123
// (causal softmax, optional softmax1 phantom term) and rows.rs:114-123 (its
// backward dx = scale y (dy - sum dy y)).  The reference materialises S and P
// ([B*H*T, T] f32 each); fusing them is the reference's own next step
// (docs/tiers_design.md:891-893).
//
// Per (window, head) problem z, with Q, K, V the head-h column blocks of the
// fused [B*T, 3D] buffer and scale = hd^-1/2:
//   forward   P = softmax(scale Q K^T, causal), O = P V, L = log-sum-exp of
//             each row (max + log(sum)), written to ctx [B*T, D] and lse [B*H*T];
//   backward  P = exp(scale S - L) recomputed, dV = P^T dO, dP = dO V^T,
//             dS = scale P (dP - D) with D = rowsum(dO o O), dQ = dS K,
//             dK = dS^T Q, written to the three blocks of dqkv [B*T, 3D].
// f16 operands (RNE from f32, as the f16 GEMM route rounds) on
// v_mfma_f32_16x16x32_f16 with f32 accumulation; softmax arithmetic in f32,
// on 2^x of scores pre-multiplied by scale log2(e) (the transcendental unit's
// exp2; lse is stored in natural-log units).
//
// Design.  T <= 256 (T % 32 == 0) and hd = 64, so a problem's operands fit on
// chip.  Work unit = one wave, which owns one 16-row block j of its problem
// (NB = T / 16 waves per workgroup, one workgroup per problem and role):
//   forward   query block j; S^T = K Q^T is computed so that each lane owns
//             one query column (row statistics need two shuffles), and its P^T
//             tiles are directly the B operand of O^T = V^T P^T;
//   backward  key block j computes dK, dV (each lane owns one key column of
//             S = Q K^T and dP = dO V^T; P and dS are the B operands of
//             dV^T = dO^T P and dK^T = Q^T dS); query block j computes dQ
//             (lane owns a query column of S^T and dP^T; dS^T is the B operand
//             of dQ^T = K^T dS^T).  No dS round trip through memory or LDS.
// A workgroup first loads its waves' own fragments, then stages the operands
// its waves share into LDS as f16 (row-major and, where an operand is needed
// transposed, V^T, Q^T, dO^T or K^T) once per problem, with every load of a
// thread in flight at once; the MFMA loops then read only LDS and registers.
// Causal work is uneven across the waves (block j has j + 1 tiles); at T = 128
// two waves share a SIMD, and the backward gives them blocks p and NB - 1 - p
// so that every SIMD carries the same number of tile pairs (block_of).  The
// outputs leave through nontemporal stores, so that they stream out as the
// waves finish rather than wait in L2 for the end-of-kernel write-back.  Two
// 16-row tiles form the 32-deep k-chunk of an MFMA whose contraction runs over
// rows: element e of lane group g is
// row 4g + e of the first tile (e < 4) or of the second (e >= 4), the order in
// which the 16x16 accumulator layout hands them out; A and B agree on it.
#include "common.h"
#include "lanes.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int HD = 64;
constexpr int TMAX = 256;

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// 2^x on the transcendental unit (v_exp_f32); x <= 0 here, 2^-inf = 0.
__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 8 consecutive f32 (16-byte aligned) as f16, round to nearest even.
__device__ __forceinline__ half8 ld_frag(const float *p) {
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    return half8{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                 (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
}

// Shapes of a problem of T = 16 NB rows: G workgroups per problem (and
// role) of W waves, one wave per 16-row block; LDS row pitch KP for row-major
// tiles and LDT for transposed ones (8 halves of padding spread the rows over
// the LDS banks).  With G = 2 the blocks pair as (p, NB - 1 - p), whose causal
// work is NB + 1 tiles per pair, and workgroup x takes the pairs p = x, x + 2,
// .., so both carry the same work and a problem spreads over two CUs.  The
// forward splits (its 128 problems would fill half the CUs of the device);
// the backward, with two roles per problem already, does not (four
// workgroups per problem staging full panels measured slower).
template <int NB, int G_>
struct Split {
    static constexpr int G = G_;
    static constexpr int W = G == 1 ? NB : 2 * ((NB + 3) / 4);
    static constexpr int NT = 64 * W;
    static constexpr int T = NB * 16, KP = HD + 8, LDT = T + 8;
};
template <int NB>
using SplitF = Split<NB, (NB >= 4 ? 2 : 1)>;
template <int NB>
using SplitB = Split<NB, 1>;

// Block of wave w of workgroup x of a problem, or -1 (a wave without a block
// when the pairs do not split evenly).  With G = 1 the first NB / 2 waves take
// blocks 0, 1, .. and the rest take NB - 1, NB - 2, ..: a workgroup's waves are
// dealt to the CU's 4 SIMDs in turn, so for NB = 8 the two waves on a SIMD hold
// blocks p and NB - 1 - p, which carry NB / 2 + 1 tile pairs between them in
// either backward role (a SIMD's waves share its matrix core and issue slots).
template <int NB, int G>
__device__ __forceinline__ int block_of(int w, int x) {
    if constexpr (G == 1) return w < NB / 2 ? w : 3 * NB / 2 - 1 - w;
    const int p = 2 * (w >> 1) + x;
    return p < NB / 2 ? ((w & 1) ? NB - 1 - p : p) : -1;
}

// Rows [0, n) (n % 32 == 0) of x (64 columns, row stride ld floats) into LDS
// as f16: row-major xr[n][kp] and / or transposed xt[64][ldt].  Thread i
// takes columns 4 (i % 16) .. + 3 of rows 4 (i / 16) .. + 3, so 16 threads
// read each 256-byte row and a transposed store is 8 bytes (4 rows); all of a
// thread's loads are issued before its first store.  With o != nullptr (and
// y the matching rows of a second matrix, row stride ldy) it also writes
// o[r] = sum_c x[r][c] y[r][c] in f32.
template <int NT, int MAXR>
__device__ __forceinline__ void stage(const float *x, int64_t ld, int n, _Float16 *xr, int kp, _Float16 *xt, int ldt,
                                      int tid, const float *y = nullptr, int64_t ldy = 0, float *o = nullptr) {
    constexpr int PER = (MAXR * 4 + NT - 1) / NT;  // (4-row group, column chunk) items per thread
    float4 v[PER][4], w[PER][4];
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int i = tid + e * NT, r0 = (i >> 4) * 4, c = (i & 15) * 4;
        if (r0 < n) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                v[e][k] = *reinterpret_cast<const float4 *>(x + (int64_t)(r0 + k) * ld + c);
                if (o) w[e][k] = *reinterpret_cast<const float4 *>(y + (int64_t)(r0 + k) * ldy + c);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int i = tid + e * NT, r0 = (i >> 4) * 4, c = (i & 15) * 4;
        if (r0 < n) {
            half4 hv[4];
#pragma unroll
            for (int k = 0; k < 4; k++) hv[k] = half4{(_Float16)v[e][k].x, (_Float16)v[e][k].y, (_Float16)v[e][k].z,
                                                      (_Float16)v[e][k].w};
            if (xr) {
#pragma unroll
                for (int k = 0; k < 4; k++) *reinterpret_cast<half4 *>(xr + (r0 + k) * kp + c) = hv[k];
            }
            if (xt) {
#pragma unroll
                for (int cc = 0; cc < 4; cc++)
                    *reinterpret_cast<half4 *>(xt + (c + cc) * ldt + r0) = half4{hv[0][cc], hv[1][cc], hv[2][cc], hv[3][cc]};
            }
            if (o) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    float p = v[e][k].x * w[e][k].x + v[e][k].y * w[e][k].y + v[e][k].z * w[e][k].z + v[e][k].w * w[e][k].w;
                    p += st::xor_lane(p, 1, tid & 63);
                    p += st::xor_lane(p, 2, tid & 63);
                    p += st::xor_lane(p, 4, tid & 63);
                    p += st::xor_lane(p, 8, tid & 63);
                    if ((i & 15) == 0) o[r0 + k] = p;
                }
            }
        }
    }
}

// A or B operand from a row-major f16 tile: row `row`, the 8 columns 8 g + 32 c.
__device__ __forceinline__ half8 frag_r(const _Float16 *xr, int kp, int row, int c, int g) {
    return *reinterpret_cast<const half8 *>(xr + row * kp + 32 * c + 8 * g);
}

// A operand from a transposed tile: row `row` (an hd index), the 32 columns
// of tile pair m in the pair order (lane group g: columns 32m + 4g .. + 3,
// then 32m + 16 + 4g .. + 3).
__device__ __forceinline__ half8 frag_t(const _Float16 *xt, int ldt, int row, int m, int g) {
    const half4 a = *reinterpret_cast<const half4 *>(xt + row * ldt + 32 * m + 4 * g);
    const half4 b = *reinterpret_cast<const half4 *>(xt + row * ldt + 32 * m + 16 + 4 * g);
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// The LDS operands of one pair of 16-row query tiles (2 mm, 2 mm + 1) for a dK / dV wave: the
// A operands of S and dP (rows of Q and dO), of dV and dK (the pair's columns of dO^T and Q^T),
// and L (in log2 units) and D of the 8 queries a lane holds.
template <int NB>
struct KvPair {
    half8 q[4], d[4], dt[4], qt[4];
    float l[8], dd[8];
    // Tile 2 mm + w2: its S and dP A operands, L and D.
    __device__ __forceinline__ void fetch_tile(int mm, int w2, const _Float16 *sQ, const _Float16 *sO,
                                               const float *sL, const float *sD, int li, int g) {
        constexpr int KP = Split<NB, 1>::KP;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            q[2 * w2 + c] = frag_r(sQ, KP, 16 * (2 * mm + w2) + li, c, g);
            d[2 * w2 + c] = frag_r(sO, KP, 16 * (2 * mm + w2) + li, c, g);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int qq = 16 * (2 * mm + w2) + 4 * g + r;
            l[4 * w2 + r] = sL[qq];
            dd[4 * w2 + r] = sD[qq];
        }
    }
    // The pair's dV and dK A operands.
    __device__ __forceinline__ void fetch_cols(int mm, const _Float16 *sQt, const _Float16 *sOt, int li, int g) {
        constexpr int LDT = Split<NB, 1>::LDT;
#pragma unroll
        for (int ht = 0; ht < 4; ht++) {
            dt[ht] = frag_t(sOt, LDT, 16 * ht + li, mm, g);
            qt[ht] = frag_t(sQt, LDT, 16 * ht + li, mm, g);
        }
    }
    __device__ __forceinline__ void fetch(int mm, const _Float16 *sQ, const _Float16 *sO, const _Float16 *sQt,
                                          const _Float16 *sOt, const float *sL, const float *sD, int li, int g) {
        fetch_tile(mm, 0, sQ, sO, sL, sD, li, g);
        fetch_tile(mm, 1, sQ, sO, sL, sD, li, g);
        fetch_cols(mm, sQt, sOt, li, g);
    }
};

// The LDS operands of one pair of 16-row key tiles (2 mm, 2 mm + 1) for a dQ wave: the A
// operands of S^T and dP^T (rows of K and V) and of dQ (the pair's columns of K^T).
template <int NB>
struct QPair {
    half8 k[4], v[4], kt[4];
    __device__ __forceinline__ void fetch_tile(int mm, int w2, const _Float16 *sK, const _Float16 *sV, int li, int g) {
        constexpr int KP = Split<NB, 1>::KP;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            k[2 * w2 + c] = frag_r(sK, KP, 16 * (2 * mm + w2) + li, c, g);
            v[2 * w2 + c] = frag_r(sV, KP, 16 * (2 * mm + w2) + li, c, g);
        }
    }
    __device__ __forceinline__ void fetch_cols(int mm, const _Float16 *sKt, int li, int g) {
        constexpr int LDT = Split<NB, 1>::LDT;
#pragma unroll
        for (int ht = 0; ht < 4; ht++) kt[ht] = frag_t(sKt, LDT, 16 * ht + li, mm, g);
    }
    __device__ __forceinline__ void fetch(int mm, const _Float16 *sK, const _Float16 *sV, const _Float16 *sKt, int li,
                                          int g) {
        fetch_tile(mm, 0, sK, sV, li, g);
        fetch_tile(mm, 1, sK, sV, li, g);
        fetch_cols(mm, sKt, li, g);
    }
};

// Workgroup id -> (problem z, unit u in [0, U)), placing all U units of a
// problem on one XCD (workgroups are dealt to the 8 XCDs round robin), so the
// operands that both backward roles stage are read from one L2:
// id = (z / 8) 8U + 8u + z % 8.  False for the padding ids of a problem count
// that is not a multiple of 8.
__device__ __forceinline__ bool unit_of(int U, int64_t nz, int64_t &z, int &u) {
    const int id = blockIdx.x, rest = id >> 3;
    u = rest % U;
    z = (int64_t)(rest / U) * 8 + (id & 7);
    return z < nz;
}

// grid 8 G ceil(B*H / 8) (unit_of, G workgroups per problem), W waves per workgroup.
template <int NB>
__global__ __launch_bounds__(SplitF<NB>::NT) void k_attn_fwd(const float *__restrict__ qkv, float *__restrict__ ctx,
                                                            float *__restrict__ lse, int32_t h, int64_t nz,
                                                            float scale, int32_t one) {
    using S = SplitF<NB>;
    constexpr int T = S::T, KP = S::KP, LDT = S::LDT;
    const float sl2 = scale * LOG2E;
    __shared__ _Float16 sK[T * KP];
    __shared__ _Float16 sVt[HD * LDT];
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, li = lane & 15;
    int64_t z;
    int x;
    if (!unit_of(S::G, nz, z, x)) return;
    const int j = __builtin_amdgcn_readfirstlane(block_of<NB, S::G>(tid >> 6, x));  // this wave's block
    const int jj = j < 0 ? 0 : j;  // a block whose rows exist, for the loads of a wave without one
    const int64_t bb = z / h;
    const int hh = (int)(z % h);
    const int64_t D = (int64_t)h * HD, ld = 3 * D;
    const float *base = qkv + bb * T * ld + hh * HD;  // + 0: Q, + D: K, + 2D: V

    // This wave's query fragments (B operands) first, so their loads overlap the staging.
    const float *qrow = base + (int64_t)(16 * jj + li) * ld;
    const half8 q0 = ld_frag(qrow + 8 * g), q1 = ld_frag(qrow + 32 + 8 * g);
    stage<S::NT, T>(base + D, ld, T, sK, KP, nullptr, 0, tid);
    stage<S::NT, T>(base + 2 * D, ld, T, nullptr, 0, sVt, LDT, tid);
    __syncthreads();
    if (j < 0) return;

    {
        const int qb = j;
        const int q = 16 * qb + li;  // this lane's query
        // S^T over key-tile pairs (2 mm, 2 mm + 1), lane holding keys 16 kt + 4 g + r of query q,
        // kept as scale S log2(e) so that the softmax runs on 2^x.
        // The next pair's K fragments are read while this pair's products run; a pair's
        // second tile past the diagonal is computed and masked like any other.
        const int npair = qb / 2 + 1;
        f32x4 s[NB];
        float m = -__builtin_inff();
        half8 ka[4], kn[4];
#pragma unroll
        for (int e = 0; e < 4; e++) ka[e] = frag_r(sK, KP, 16 * (e >> 1) + li, e & 1, g);
#pragma unroll
        for (int mm = 0; mm < NB / 2; mm++) {
            if (mm < npair) {
                if (mm + 1 < npair) {
#pragma unroll
                    for (int e = 0; e < 4; e++) kn[e] = frag_r(sK, KP, 16 * (2 * mm + 2 + (e >> 1)) + li, e & 1, g);
                }
                f32x4 a0 = mfma(ka[0], q0, f32x4{0.f, 0.f, 0.f, 0.f});
                f32x4 a1 = mfma(ka[2], q0, f32x4{0.f, 0.f, 0.f, 0.f});
                a0 = mfma(ka[1], q1, a0);
                a1 = mfma(ka[3], q1, a1);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = 32 * mm + 4 * g + r;
                    a0[r] = key <= q ? a0[r] * sl2 : -__builtin_inff();
                    a1[r] = key + 16 <= q ? a1[r] * sl2 : -__builtin_inff();
                    m = fmaxf(m, fmaxf(a0[r], a1[r]));
                }
                s[2 * mm] = a0;
                s[2 * mm + 1] = a1;
#pragma unroll
                for (int e = 0; e < 4; e++) ka[e] = kn[e];
            }
        }
        m = fmaxf(m, st::xor_lane(m, 16, lane));
        m = fmaxf(m, st::xor_lane(m, 32, lane));
        if (one) m = fmaxf(m, 0.f);
        float sum = 0.f;
#pragma unroll
        for (int kt = 0; kt < NB; kt++) {
            if (kt < 2 * npair) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = exp2_(s[kt][r] - m);  // masked: 2^-inf = 0
                    s[kt][r] = e;
                    sum += e;
                }
            }
        }
        sum += st::xor_lane(sum, 16, lane);
        sum += st::xor_lane(sum, 32, lane);
        if (one) sum += exp2_(-m);
        const float inv = 1.f / sum;
        // O^T = V^T P^T over the same pairs, the next pair's V^T fragments read ahead.
        f32x4 o[4];
        half8 va[4], vn[4];
#pragma unroll
        for (int ht = 0; ht < 4; ht++) {
            o[ht] = f32x4{0.f, 0.f, 0.f, 0.f};
            va[ht] = frag_t(sVt, LDT, 16 * ht + li, 0, g);
        }
#pragma unroll
        for (int mm = 0; mm < NB / 2; mm++) {
            if (mm < npair) {
                if (mm + 1 < npair) {
#pragma unroll
                    for (int ht = 0; ht < 4; ht++) vn[ht] = frag_t(sVt, LDT, 16 * ht + li, mm + 1, g);
                }
                half8 pb;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    pb[r] = (_Float16)(s[2 * mm][r] * inv);
                    pb[4 + r] = (_Float16)(s[2 * mm + 1][r] * inv);
                }
#pragma unroll
                for (int ht = 0; ht < 4; ht++) o[ht] = mfma(va[ht], pb, o[ht]);
#pragma unroll
                for (int ht = 0; ht < 4; ht++) va[ht] = vn[ht];
            }
        }
        float *orow = ctx + (bb * T + q) * D + hh * HD;
#pragma unroll
        for (int ht = 0; ht < 4; ht++) __builtin_nontemporal_store(o[ht], reinterpret_cast<f32x4 *>(orow + 16 * ht + 4 * g));
        if (g == 0) lse[z * T + q] = (m + __log2f(sum)) * LN2;
    }
}

// grid 16 G ceil(B*H / 8) (unit_of, 2 G workgroups per problem: G computing
// dK, dV by key block, G computing dQ by query block), W waves per workgroup.
template <int NB>
__global__ __launch_bounds__(SplitB<NB>::NT) void k_attn_bwd(const float *__restrict__ qkv,
                                                            const float *__restrict__ ctx,
                                                            const float *__restrict__ dctx,
                                                            const float *__restrict__ lse, float *__restrict__ dqkv,
                                                            int32_t h, int64_t nz, float scale) {
    using S = SplitB<NB>;
    constexpr int T = S::T, KP = S::KP, LDT = S::LDT;
    // Each wave reads the next tile pair's LDS operands while it multiplies the current one, where
    // the registers allow: up to 8 waves a workgroup (2 a SIMD); more waves would spill them.
    constexpr bool PF = NB <= 8;
    const float sl2 = scale * LOG2E;
    // dK/dV units: Q, dO row-major, Q^T, dO^T; dQ units: K, V row-major, K^T.
    __shared__ _Float16 sR0[T * KP], sR1[T * KP];
    __shared__ _Float16 sT0[HD * LDT], sT1[HD * LDT];
    __shared__ float sL[T], sD[T];
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, li = lane & 15;
    int64_t z;
    int x;
    if (!unit_of(2 * S::G, nz, z, x)) return;
    const bool kv = x < S::G;
    const int j = __builtin_amdgcn_readfirstlane(block_of<NB, S::G>(tid >> 6, kv ? x : x - S::G));  // this wave's block
    const int jj = j < 0 ? 0 : j;  // a block whose rows exist, for the loads of a wave without one
    const int64_t bb = z / h;
    const int hh = (int)(z % h);
    const int64_t D = (int64_t)h * HD, ld = 3 * D;
    const float *base = qkv + bb * T * ld + hh * HD;
    const float *obase = ctx + bb * T * D + hh * HD;
    const float *dobase = dctx + bb * T * D + hh * HD;
    float *gbase = dqkv + bb * T * ld + hh * HD;
    const float *lrow = lse + z * T;

    if (kv) {
        // This wave's key and value fragments (B operands) first.
        const float *krow = base + D + (int64_t)(16 * jj + li) * ld, *vrow = krow + D;
        const half8 k0 = ld_frag(krow + 8 * g), k1 = ld_frag(krow + 32 + 8 * g);
        const half8 v0 = ld_frag(vrow + 8 * g), v1 = ld_frag(vrow + 32 + 8 * g);
        // Q, dO (row-major and transposed), L and D = rowsum(dO o O) of every query.
        stage<S::NT, T>(base, ld, T, sR0, KP, sT0, LDT, tid);
        stage<S::NT, T>(dobase, D, T, sR1, KP, sT1, LDT, tid, obase, D, sD);
        for (int r = tid; r < T; r += S::NT) sL[r] = lrow[r] * LOG2E;
        __syncthreads();
        if (j < 0) return;
        {
            const int kb = j;
            const int key = 16 * kb + li;  // this lane's key
            f32x4 dv[4], dk[4];
#pragma unroll
            for (int ht = 0; ht < 4; ht++) dv[ht] = dk[ht] = f32x4{0.f, 0.f, 0.f, 0.f};
            // Query-tile pairs NB/2 - 1 down to m0 (tiles 2 mm, 2 mm + 1; a tile before the key
            // block masks to zero), so every wave starts on the same code; each pair's LDS
            // operands are read while the pair before it runs (buffer i % 2 holds the i-th).
            const int m0 = kb >> 1;
            KvPair<NB> f[PF ? 2 : 1];
            if constexpr (PF) f[0].fetch(NB / 2 - 1, sR0, sR1, sT0, sT1, sL, sD, li, g);
#pragma unroll
            for (int i = 0; i < NB / 2; i++) {
                const int mm = NB / 2 - 1 - i;
                if (mm < m0) break;
                KvPair<NB> &c = f[PF ? (i & 1) : 0];
                if constexpr (PF) {
                    if (mm - 1 >= m0) f[(i + 1) & 1].fetch(mm - 1, sR0, sR1, sT0, sT1, sL, sD, li, g);
                }
                half8 pb, sb;
#pragma unroll
                for (int w2 = 0; w2 < 2; w2++) {
                    if constexpr (!PF) c.fetch_tile(mm, w2, sR0, sR1, sL, sD, li, g);
                    // S = Q K^T and dP = dO V^T: lane holds queries 16 qt + 4 g + r of its key.
                    f32x4 sv = mfma(c.q[2 * w2], k0, f32x4{0.f, 0.f, 0.f, 0.f});
                    sv = mfma(c.q[2 * w2 + 1], k1, sv);
                    f32x4 dp = mfma(c.d[2 * w2], v0, f32x4{0.f, 0.f, 0.f, 0.f});
                    dp = mfma(c.d[2 * w2 + 1], v1, dp);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int q = 16 * (2 * mm + w2) + 4 * g + r;
                        const float p = key <= q ? exp2_(fmaf(sv[r], sl2, -c.l[4 * w2 + r])) : 0.f;
                        pb[4 * w2 + r] = (_Float16)p;
                        sb[4 * w2 + r] = (_Float16)(p * (dp[r] - c.dd[4 * w2 + r]) * scale);
                    }
                }
                if constexpr (!PF) c.fetch_cols(mm, sT0, sT1, li, g);
#pragma unroll
                for (int ht = 0; ht < 4; ht++) {
                    dv[ht] = mfma(c.dt[ht], pb, dv[ht]);
                    dk[ht] = mfma(c.qt[ht], sb, dk[ht]);
                }
            }
            float *gr = gbase + (int64_t)key * ld;
#pragma unroll
            for (int ht = 0; ht < 4; ht++) {
                __builtin_nontemporal_store(dk[ht], reinterpret_cast<f32x4 *>(gr + D + 16 * ht + 4 * g));
                __builtin_nontemporal_store(dv[ht], reinterpret_cast<f32x4 *>(gr + 2 * D + 16 * ht + 4 * g));
            }
        }
    } else {
        // This wave's query and upstream-gradient fragments (B operands), D and
        // L of its queries first, so their loads overlap the staging.
        half8 q0, q1, d0, d1;
        float dsum = 0.f, L;
        {
            const int64_t q = 16 * jj + li;
            const float *qr = base + q * ld, *dr = dobase + q * D, *orr = obase + q * D;
            float4 dv[4], ov[4];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                dv[2 * c] = *reinterpret_cast<const float4 *>(dr + 32 * c + 8 * g);
                dv[2 * c + 1] = *reinterpret_cast<const float4 *>(dr + 32 * c + 8 * g + 4);
                ov[2 * c] = *reinterpret_cast<const float4 *>(orr + 32 * c + 8 * g);
                ov[2 * c + 1] = *reinterpret_cast<const float4 *>(orr + 32 * c + 8 * g + 4);
            }
            q0 = ld_frag(qr + 8 * g);
            q1 = ld_frag(qr + 32 + 8 * g);
            d0 = half8{(_Float16)dv[0].x, (_Float16)dv[0].y, (_Float16)dv[0].z, (_Float16)dv[0].w,
                       (_Float16)dv[1].x, (_Float16)dv[1].y, (_Float16)dv[1].z, (_Float16)dv[1].w};
            d1 = half8{(_Float16)dv[2].x, (_Float16)dv[2].y, (_Float16)dv[2].z, (_Float16)dv[2].w,
                       (_Float16)dv[3].x, (_Float16)dv[3].y, (_Float16)dv[3].z, (_Float16)dv[3].w};
#pragma unroll
            for (int k = 0; k < 4; k++) dsum += dv[k].x * ov[k].x + dv[k].y * ov[k].y + dv[k].z * ov[k].z + dv[k].w * ov[k].w;
            dsum += st::xor_lane(dsum, 16, lane);
            dsum += st::xor_lane(dsum, 32, lane);
            L = lrow[q] * LOG2E;
        }
        // K (row-major and transposed) and V of every key.
        stage<S::NT, T>(base + D, ld, T, sR0, KP, sT0, LDT, tid);
        stage<S::NT, T>(base + 2 * D, ld, T, sR1, KP, nullptr, 0, tid);
        __syncthreads();
        if (j < 0) return;
        {
            const int qb = j;
            const int q = 16 * qb + li;  // this lane's query
            f32x4 dq[4];
#pragma unroll
            for (int ht = 0; ht < 4; ht++) dq[ht] = f32x4{0.f, 0.f, 0.f, 0.f};
            // Key-tile pairs 0 .. qb / 2 (a tile past the query block masks to zero), each
            // pair's LDS operands read while the pair before it runs: buffer mm % 2 holds pair mm.
            const int m1 = qb >> 1;
            QPair<NB> f[PF ? 2 : 1];
            if constexpr (PF) f[0].fetch(0, sR0, sR1, sT0, li, g);
#pragma unroll
            for (int mm = 0; mm < NB / 2; mm++) {
                if (mm > m1) break;
                QPair<NB> &c = f[PF ? (mm & 1) : 0];
                if constexpr (PF) {
                    if (mm + 1 < NB / 2 && mm + 1 <= m1) f[(mm + 1) & 1].fetch(mm + 1, sR0, sR1, sT0, li, g);
                }
                half8 sb;
#pragma unroll
                for (int w2 = 0; w2 < 2; w2++) {
                    if constexpr (!PF) c.fetch_tile(mm, w2, sR0, sR1, li, g);
                    // S^T = K Q^T and dP^T = V dO^T: lane holds keys 16 kt + 4 g + r of its query.
                    f32x4 st = mfma(c.k[2 * w2], q0, f32x4{0.f, 0.f, 0.f, 0.f});
                    st = mfma(c.k[2 * w2 + 1], q1, st);
                    f32x4 dpt = mfma(c.v[2 * w2], d0, f32x4{0.f, 0.f, 0.f, 0.f});
                    dpt = mfma(c.v[2 * w2 + 1], d1, dpt);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int key = 16 * (2 * mm + w2) + 4 * g + r;
                        const float p = key <= q ? exp2_(fmaf(st[r], sl2, -L)) : 0.f;
                        sb[4 * w2 + r] = (_Float16)(p * (dpt[r] - dsum) * scale);
                    }
                }
                if constexpr (!PF) c.fetch_cols(mm, sT0, li, g);
#pragma unroll
                for (int ht = 0; ht < 4; ht++) dq[ht] = mfma(c.kt[ht], sb, dq[ht]);
            }
            float *gr = gbase + (int64_t)q * ld;
#pragma unroll
            for (int ht = 0; ht < 4; ht++) __builtin_nontemporal_store(dq[ht], reinterpret_cast<f32x4 *>(gr + 16 * ht + 4 * g));
        }
    }
}

template <int NB>
void launch_fwd(const float *qkv, float *ctx, float *lse, int64_t b, int64_t h, float scale, int32_t one,
                hipStream_t s) {
    const int64_t nz = b * h;
    hipLaunchKernelGGL(k_attn_fwd<NB>, dim3((unsigned)(8 * SplitF<NB>::G * ((nz + 7) / 8))), dim3(SplitF<NB>::NT), 0, s,
                       qkv, ctx, lse, (int32_t)h, nz, scale, one);
}

template <int NB>
void launch_bwd(const float *qkv, const float *ctx, const float *dctx, const float *lse, float *dqkv, int64_t b,
                int64_t h, float scale, hipStream_t s) {
    const int64_t nz = b * h;
    hipLaunchKernelGGL(k_attn_bwd<NB>, dim3((unsigned)(16 * SplitB<NB>::G * ((nz + 7) / 8))), dim3(SplitB<NB>::NT), 0,
                       s, qkv, ctx, dctx, lse, dqkv, (int32_t)h, nz, scale);
}

st_status check_shape(const char *what, int64_t b, int64_t h, int64_t t, int64_t hd) {
    if (hd != HD) return st::fail(ST_ERR_INVALID, "%s: the fused attention is built for head_dim %d (got %lld)", what,
                                  HD, (long long)hd);
    if (t < 32 || t > TMAX || t % 32 != 0)
        return st::fail(ST_ERR_INVALID, "%s: seq_len must be a multiple of 32 in 32..=%d (got %lld)", what, TMAX,
                        (long long)t);
    if (b < 1 || h < 1 || b * h > (1 << 24) || h * 3 * HD > INT32_MAX)
        return st::fail(ST_ERR_INVALID, "%s: bad batch or head count", what);
    return ST_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" st_status st_attention_fused_fwd(const float *qkv, float *ctx, float *lse, int64_t b, int64_t h, int64_t t,
                                            int64_t hd, float scale, int32_t one, st_stream stream) {
    st::clear_error();
    if (!qkv || !ctx || !lse) return st::fail(ST_ERR_INVALID, "attention_fused_fwd: NULL buffer");
    st_status st = check_shape("attention_fused_fwd", b, h, t, hd);
    if (st != ST_OK) return st;
    if (!aligned16(qkv) || !aligned16(ctx))
        return st::fail(ST_ERR_INVALID, "attention_fused_fwd: qkv and ctx must be 16-byte aligned");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const hipStream_t s = st::stream_of(stream);
    switch (t / 16) {
        case 2: launch_fwd<2>(qkv, ctx, lse, b, h, scale, one, s); break;
        case 4: launch_fwd<4>(qkv, ctx, lse, b, h, scale, one, s); break;
        case 6: launch_fwd<6>(qkv, ctx, lse, b, h, scale, one, s); break;
        case 8: launch_fwd<8>(qkv, ctx, lse, b, h, scale, one, s); break;
        case 10: launch_fwd<10>(qkv, ctx, lse, b, h, scale, one, s); break;
        case 12: launch_fwd<12>(qkv, ctx, lse, b, h, scale, one, s); break;
        case 14: launch_fwd<14>(qkv, ctx, lse, b, h, scale, one, s); break;
        default: launch_fwd<16>(qkv, ctx, lse, b, h, scale, one, s); break;
    }
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_attention_fused_bwd(const float *qkv, const float *ctx, const float *dctx, const float *lse,
                                            float *dqkv, int64_t b, int64_t h, int64_t t, int64_t hd, float scale,
                                            st_stream stream) {
    st::clear_error();
    if (!qkv || !ctx || !dctx || !lse || !dqkv) return st::fail(ST_ERR_INVALID, "attention_fused_bwd: NULL buffer");
    st_status st = check_shape("attention_fused_bwd", b, h, t, hd);
    if (st != ST_OK) return st;
    if (!aligned16(qkv) || !aligned16(ctx) || !aligned16(dctx) || !aligned16(dqkv))
        return st::fail(ST_ERR_INVALID, "attention_fused_bwd: qkv, ctx, dctx and dqkv must be 16-byte aligned");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const hipStream_t s = st::stream_of(stream);
    switch (t / 16) {
        case 2: launch_bwd<2>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
        case 4: launch_bwd<4>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
        case 6: launch_bwd<6>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
        case 8: launch_bwd<8>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
        case 10: launch_bwd<10>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
        case 12: launch_bwd<12>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
        case 14: launch_bwd<14>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
        default: launch_bwd<16>(qkv, ctx, dctx, lse, dqkv, b, h, scale, s); break;
    }
    ST_LAUNCH_CHECK();
    return ST_OK;
}
