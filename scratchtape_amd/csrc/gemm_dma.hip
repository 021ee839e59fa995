// GEMM on gfx950 with operand tiles moved global -> LDS by the DMA path of
// global_load_lds_dwordx4: no register staging, NS - 1 k-stages in flight, one
// barrier per stage.  f16-in/f32-accumulate (v_mfma_f32_32x32x16_f16, f32
// rounded to f16 to nearest even when a fragment is read from LDS; on gfx950
// it does twice the work of v_mfma_f32_16x16x32_f16 per issue) and f32
// (v_mfma_f32_16x16x4_f32).  Semantics: gpu_step/matmul.rs:26-299 (MatRef
// addressing, the epilogue in the reference's order, deterministic split-k).
//
// LDS layouts and the DMA / wait / barrier helpers: dma_tile.h.
//
// The finished tile goes through LDS once more so that every store (and every
// epilogue load) moves whole 16-byte runs of a row.  Split-k (few output
// tiles, free epilogue): each slice writes its partial tile to the scratch
// arena and k_sum_slices adds the slices in ascending order (deterministic),
// with accumulate and the column sums, as the reference's k_split_sum
// (matmul.rs:259-299).
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "dma_tile.h"
#include "gemm_dma.h"

namespace {

using namespace dma;

constexpr int THREADS = 256;

struct KArgs {
    const float *a, *b;
    int64_t a_stride, a_group, a_inner, lda;
    int64_t b_stride, b_group, b_inner, ldb;
    float *out;  // the output, or the split partials [batch][splits][m][n]
    int64_t o_stride, o_group, o_inner, ldo;
    const float *bias;
    int64_t bias_stride;
    const float *mask, *res;
    float *cs;  // column-sum destination (out buffer + col_sum_off), or the split partials
    int64_t cs_stride;
    int32_t has_cs, relu, accumulate;
    int32_t m, n, k, splits, slice_k;
};

// NS k-stages resident in LDS, NS - 1 of them in flight while one is multiplied.
template <int BM, int BN, int NS, bool TA, bool TB, bool F16>
__global__ __launch_bounds__(THREADS) void k_gemm_dma(KArgs g) {
    constexpr bool AKC = !TA, BKC = TB;
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int LA = BM / 32, LB = BN / 32;  // DMA wave-loads per wave per stage
    constexpr int SA = BM * BK, SB = BN * BK;  // floats per stage
    // Row pitch of the staged output tile: 16 banks between the 4-row groups of
    // a 16 x 16 block, 32 between the two lane halves of a 32 x 32 block.
    constexpr int TP = F16 ? BN + 8 : BN + 4;
    constexpr int M32 = WM / 32, N32 = WN / 32;
    static_assert(!F16 || (M32 >= 1 && N32 >= 1), "32 x 32 blocks per wave");
    static_assert(BM * TP <= NS * (SA + SB), "output tile fits the stage ring");
    __shared__ __attribute__((aligned(16))) float lds[NS * (SA + SB)];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // Workgroups go to the 8 XCDs round-robin by linear id: remap so each XCD
    // gets a contiguous run of tiles (sharing operand panels in its L2).
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
    const int nst = (kend - kbeg) / BK;
    const bool do_cs = g.has_cs && by == 0;

    const float *abase = g.a + zoff(zb, g.a_group, g.a_stride, g.a_inner);
    const float *bbase = g.b + zoff(zb, g.b_group, g.b_stride, g.b_inner);
    int64_t aoff[LA], boff[LB];
#pragma unroll
    for (int j = 0; j < LA; j++)
        aoff[j] = slot_src<BM, AKC>((wave * LA + j) * 64 + lane, g.lda, row0) + (AKC ? kbeg : (int64_t)kbeg * g.lda);
#pragma unroll
    for (int j = 0; j < LB; j++)
        boff[j] = slot_src<BN, BKC>((wave * LB + j) * 64 + lane, g.ldb, col0) + (BKC ? kbeg : (int64_t)kbeg * g.ldb);
    const int64_t astep = AKC ? BK : (int64_t)BK * g.lda, bstep = BKC ? BK : (int64_t)BK * g.ldb;

    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    auto issue = [&](int st) {
        const uint32_t base = lds_addr_of(lds + (st % NS) * (SA + SB));
#pragma unroll
        for (int j = 0; j < LA; j++) dma16(abase + aoff[j] + st * astep, base + (wave_u * LA + j) * 1024);
#pragma unroll
        for (int j = 0; j < LB; j++) dma16(bbase + boff[j] + st * bstep, base + SA * 4 + (wave_u * LB + j) * 1024);
    };

    constexpr int AM = M32 > 0 ? M32 : 1, AN = N32 > 0 ? N32 : 1;  // (32 x 32 f32 tiles have no 32 x 32 blocks)
    f32x4 acc[FM][FN];    // f32 route: 16 x 16 blocks
    f32x16 acc2[AM][AN];  // f16 route: 32 x 32 blocks
    if constexpr (F16) {
#pragma unroll
        for (int i = 0; i < M32; i++)
#pragma unroll
            for (int j = 0; j < N32; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc2[i][j][e] = 0.f;
    } else {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float cs_acc = 0.f;  // column sum of B for column col0 + tid (tid < BN), this slice

    // Stage st lives in ring slot st % NS.  Per stage: wait for this wave's DMA
    // of stage st (younger stages stay in flight), barrier (every wave's part
    // of stage st has landed, and every wave is done reading stage st - 1),
    // start stage st + NS - 1 into stage st - 1's slot, multiply stage st.
    auto step = [&](int st) {
        wait_stage<LA + LB, NS - 2>(min(NS - 2, nst - 1 - st));
        bar();
        if (st + NS - 1 < nst) issue(st + NS - 1);
        const float *la = lds + (st % NS) * (SA + SB);
        const float *lb = la + SA;
        const int gq = lane >> 4;
        if constexpr (F16) {
            // 32 x 32 x 16 operands: lane l holds row (or column) l % 32 and
            // the 8 k of group 2 ks + l / 32 of the stage.
            half8 af[M32][2], bf[N32][2];
            const int r32 = lane & 31, h = lane >> 5;
#pragma unroll
            for (int i = 0; i < M32; i++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    float x[8];
                    frag<BM, AKC>(la, wm * WM + i * 32 + r32, 2 * ks + h, x);
#pragma unroll
                    for (int e = 0; e < 8; e++) af[i][ks][e] = (_Float16)x[e];
                }
#pragma unroll
            for (int j = 0; j < N32; j++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    float x[8];
                    frag<BN, BKC>(lb, wn * WN + j * 32 + r32, 2 * ks + h, x);
#pragma unroll
                    for (int e = 0; e < 8; e++) bf[j][ks][e] = (_Float16)x[e];
                }
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int i = 0; i < M32; i++)
#pragma unroll
                    for (int j = 0; j < N32; j++)
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][ks], bf[j][ks], acc2[i][j], 0, 0, 0);
        } else {
            // Lane group gq supplies k = 8 gq + u at MFMA step u, for A and B alike.
            float ax[FM][8], bx8[FN][8];
#pragma unroll
            for (int i = 0; i < FM; i++) frag<BM, AKC>(la, wm * WM + i * 16 + (lane & 15), gq, ax[i]);
#pragma unroll
            for (int j = 0; j < FN; j++) frag<BN, BKC>(lb, wn * WN + j * 16 + (lane & 15), gq, bx8[j]);
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(ax[i][u], bx8[j][u], acc[i][j], 0, 0, 0);
        }
        if (do_cs && tid < BN) {
            // This stage's 32 values of column col0 + tid in k order: f32 route
            // one running sum; f16 route, the sum of each 8 consecutive k
            // (from 0, in order) added in order, as the grouped f16 kernel sums
            // the columns (each of its lanes holds 8 consecutive k of a column).
            float x[8];
#pragma unroll
            for (int gg = 0; gg < 4; gg++) {
                frag<BN, BKC>(lb, tid, gg, x);
                if constexpr (F16) {
                    float p = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; e++) p += x[e];
                    cs_acc += p;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) cs_acc += x[e];
                }
            }
        }
    };

#pragma unroll
    for (int st = 0; st < NS - 1; st++)
        if (st < nst) issue(st);
    for (int st = 0; st < nst; st++) step(st);

    if (do_cs && tid < BN) {
        if (g.splits > 1)
            g.cs[(zb * g.splits + slice) * (int64_t)g.n + col0 + tid] = cs_acc;
        else
            g.cs[zb * g.cs_stride + col0 + tid] += cs_acc;
    }

    // Output tile -> LDS (row pitch TP: the 16 lanes of a row write 16
    // consecutive words and the 4 row groups land 16 banks apart) -> whole
    // 16-byte runs of rows to memory, with the epilogue in the reference's
    // order: + bias, ReLU, zero where mask <= 0, + residual, + out.
    bar();  // every wave is done with the stage ring
    if constexpr (F16) {
        // Element e of a lane of a 32 x 32 block: row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32.
#pragma unroll
        for (int i = 0; i < M32; i++)
#pragma unroll
            for (int j = 0; j < N32; j++)
#pragma unroll
                for (int e = 0; e < 16; e++)
                    lds[(wm * WM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * TP + wn * WN + j * 32 +
                        (lane & 31)] = acc2[i][j][e];
    } else {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    lds[(wm * WM + i * 16 + 4 * (lane >> 4) + r) * TP + wn * WN + j * 16 + (lane & 15)] = acc[i][j][r];
    }
    bar();
    if (g.splits > 1) {
        float *P = g.out + (zb * g.splits + slice) * (int64_t)g.m * g.n;
        for (int e = tid; e < BM * BN / 4; e += THREADS) {
            const int r = e / (BN / 4), c4 = (e % (BN / 4)) * 4;
            *reinterpret_cast<f32x4 *>(P + (int64_t)(row0 + r) * g.n + col0 + c4) =
                *reinterpret_cast<const f32x4 *>(lds + r * TP + c4);
        }
        return;
    }
    const int64_t o0 = zoff(zb, g.o_group, g.o_stride, g.o_inner);
    for (int e = tid; e < BM * BN / 4; e += THREADS) {
        const int r = e / (BN / 4), c4 = (e % (BN / 4)) * 4;
        f32x4 v = *reinterpret_cast<const f32x4 *>(lds + r * TP + c4);
        const int col = col0 + c4;
        const int64_t idx = o0 + (int64_t)(row0 + r) * g.ldo + col;
        if (g.bias) {
            const float *bp = g.bias + zb * g.bias_stride + col;
#pragma unroll
            for (int x = 0; x < 4; x++) v[x] += bp[x];
        }
        if (g.relu) {
#pragma unroll
            for (int x = 0; x < 4; x++)
                if (v[x] < 0.f) v[x] = 0.f;
        }
        if (g.mask) {
            const f32x4 mk = *reinterpret_cast<const f32x4 *>(g.mask + idx);
#pragma unroll
            for (int x = 0; x < 4; x++)
                if (mk[x] <= 0.f) v[x] = 0.f;
        }
        if (g.res) v += *reinterpret_cast<const f32x4 *>(g.res + idx);
        if (g.accumulate) v += *reinterpret_cast<const f32x4 *>(g.out + idx);
        *reinterpret_cast<f32x4 *>(g.out + idx) = v;
    }
}

// out[b] (+)= sum over s (ascending) of partial[b][s], 4 elements per thread;
// then the column-sum partials into their destination (always +=).  Each
// thread's slice loads are in flight together (sum_slices).
__global__ __launch_bounds__(256) void k_sum_slices(const float *__restrict__ part, float *out, int64_t mn,
                                                    int32_t splits, int64_t o_stride, int64_t batch,
                                                    int32_t accumulate, const float *cs_part, float *cs_dst,
                                                    int64_t cs_stride, int64_t n) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t q = mn / 4;
    if (e < batch * q) {
        const int64_t b = batch == 1 ? 0 : e / q, i = batch == 1 ? e : e % q;
        const f32x4 *p = reinterpret_cast<const f32x4 *>(part) + b * splits * q + i;
        f32x4 v = sum_slices(p, q, splits, f32x4{0.f, 0.f, 0.f, 0.f});
        f32x4 *o = reinterpret_cast<f32x4 *>(out + b * o_stride) + i;
        if (accumulate) v += *o;
        *o = v;
    } else if (cs_part) {
        const int64_t c = e - batch * q;
        if (c < batch * n) {
            const int64_t b = c / n, j = c % n;
            const float v = sum_slices(cs_part + b * splits * n + j, n, splits, 0.f);
            cs_dst[b * cs_stride + j] += v;
        }
    }
}

// Small products (no column sums, m % 16 = n % 16 = 0, k % 256 = 0, so each
// wave's quarter of k is whole passes of 64): one 16 x 16 output tile per
// workgroup, so that a 256 x 256
// product spreads over 256 CUs (32 x 32 tiles leave 64 of them 0.85 us of
// matrix-core work each).  The four waves split k into quarters, taken in
// passes of 64; in a pass lane group q (lanes 16 q .. 16 q + 15) holds k
// p0 + 16 q .. + 15 of its A row and B column, so MFMA step j sums k
// {p0 + j, p0 + 16 + j, p0 + 32 + j, p0 + 48 + j}.  Every load of a pass is
// issued before the first MFMA.  The waves' partial tiles are added in wave
// order through LDS (deterministic), then the epilogue in the reference's
// order.  f32 route: v_mfma_f32_16x16x4_f32, one k per lane group and step;
// f16 route: the operands rounded to f16 (nearest even) and two
// v_mfma_f32_16x16x32_f16 per pass, element e of the lane's 16 k in the
// first (e < 8) or second instruction (A and B agree on the order).  Lane l
// ends with rows 4 (l / 16) + e, column l % 16 of the tile.
template <bool TA, bool TB, bool F16>
__global__ __launch_bounds__(256) void k_gemm_tiny(KArgs g) {
    __shared__ f32x4 part[3][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int64_t zb = blockIdx.z;
    const int row0 = blockIdx.y * 16, col0 = blockIdx.x * 16;
    const float *A = g.a + zoff(zb, g.a_group, g.a_stride, g.a_inner);
    const float *B = g.b + zoff(zb, g.b_group, g.b_stride, g.b_inner);
    const int kq = g.k / 4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int p0 = wave * kq; p0 < (wave + 1) * kq; p0 += 64) {
        const int kb = p0 + 16 * q;
        float a[16], b[16];
        if constexpr (!TA) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(A + (int64_t)(row0 + r) * g.lda + kb + 4 * i);
#pragma unroll
                for (int e = 0; e < 4; e++) a[4 * i + e] = v[e];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) a[j] = A[(int64_t)(kb + j) * g.lda + row0 + r];
        }
        if constexpr (TB) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(B + (int64_t)(col0 + r) * g.ldb + kb + 4 * i);
#pragma unroll
                for (int e = 0; e < 4; e++) b[4 * i + e] = v[e];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) b[j] = B[(int64_t)(kb + j) * g.ldb + col0 + r];
        }
        if constexpr (F16) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                half8 ah, bh;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    ah[e] = (_Float16)a[8 * h + e];
                    bh[e] = (_Float16)b[8 * h + e];
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], acc, 0, 0, 0);
        }
    }
    if (wave > 0) part[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0) return;
    acc = ((acc + part[0][lane]) + part[1][lane]) + part[2][lane];
    const int64_t o0 = zoff(zb, g.o_group, g.o_stride, g.o_inner);
    const int col = col0 + r;
    const float bv = g.bias ? g.bias[zb * g.bias_stride + col] : 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int64_t idx = o0 + (int64_t)(row0 + 4 * q + e) * g.ldo + col;
        float v = acc[e];
        if (g.bias) v += bv;
        if (g.relu && v < 0.f) v = 0.f;
        if (g.mask && g.mask[idx] <= 0.f) v = 0.f;
        if (g.res) v += g.res[idx];
        if (g.accumulate) v += g.out[idx];
        g.out[idx] = v;
    }
}

using KernelFn = void (*)(KArgs);

template <int BM, int BN, int NS, bool F16>
KernelFn pick(bool ta, bool tb) {
    if (!ta && !tb) return &k_gemm_dma<BM, BN, NS, false, false, F16>;
    if (!ta && tb) return &k_gemm_dma<BM, BN, NS, false, true, F16>;
    if (ta && !tb) return &k_gemm_dma<BM, BN, NS, true, false, F16>;
    return &k_gemm_dma<BM, BN, NS, true, true, F16>;
}

template <int BM, int BN, int NS>
KernelFn pick2(bool f16, bool ta, bool tb) {
    return f16 ? pick<BM, BN, NS, true>(ta, tb) : pick<BM, BN, NS, false>(ta, tb);
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The kernel's tile and split-k for d; false when the kernel does not take d.
struct DmaPlan {
    int bm, bn;
    int64_t splits, slice_k;
    bool tiny;  // k_gemm_tiny instead of k_gemm_dma
};

bool dma_plan(const st::DmaGemm &d, DmaPlan &p) {
    const int64_t m = d.m, n = d.n, k = d.k, batch = d.batch;
    if (k <= 0 || k % BK != 0) return false;
    // 16-byte runs everywhere: operands for the DMA, out / mask / residual for
    // the vector epilogue.
    if (!al16(d.a) || !al16(d.b) || d.lda % 4 || d.ldb % 4 || d.a_stride % 4 || d.a_inner % 4 || d.b_stride % 4 ||
        d.b_inner % 4)
        return false;
    if (!al16(d.out) || d.ldo % 4 || d.o_stride % 4 || d.o_inner % 4 || (d.mask && !al16(d.mask)) ||
        (d.res && !al16(d.res)))
        return false;
    // Split-k only as the reference allows it (matmul.rs:117-123): no epilogue
    // but +=, out packed.
    const bool can_split = !d.bias && !d.relu && !d.mask && !d.res && d.ldo == n && d.o_group == 1 &&
                           (batch == 1 || d.o_stride == m * n);
    // Output tile and split count by a rough time estimate: operand panels
    // re-read from L2 per tile (~25 TB/s, stretched when fewer than 256
    // workgroups run), plus the split partials written and summed (~5 TB/s).
    struct Cfg {
        int bm, bn;
    };
    // 32 x 32 (f32 route only: the f16 route's MFMA blocks are 32 x 32 per
    // wave) spreads a small product over 4x the workgroups of 64 x 64.
    const Cfg cands[] = {{128, 128}, {128, 64}, {64, 64}, {32, 32}};
    int best = -1;
    int64_t best_splits = 1;
    double best_t = 0;
    for (int c = 0; c < 4; c++) {
        const int bm = cands[c].bm, bn = cands[c].bn;
        if (m % bm || n % bn || (bm == 32 && d.f16)) continue;
        const int64_t tiles = batch * (m / bm) * (n / bn);
        for (int64_t sp = 1; sp <= 32; sp *= 2) {
            if (sp > 1 && (!can_split || k / sp < 4 * BK)) break;
            const int64_t slice = cdiv(cdiv(k, sp), BK) * BK;
            const int64_t splits = cdiv(k, slice);
            const double wgs = (double)(tiles * splits);
            double t = 4.0 * batch * m * n * k * (1.0 / bn + 1.0 / bm) / 25e12 * std::max(1.0, 256.0 / wgs);
            if (splits > 1) t += 12.0 * splits * batch * m * n / 5e12 + 2e-6;
            if (best < 0 || t < best_t) {
                best = c;
                best_splits = splits;
                best_t = t;
            }
        }
    }
    // A small product (at most 1,024 tiles of 16 x 16, k <= 1,024, no column
    // sums) that no tile fits, or whose best tiling leaves most CUs idle,
    // takes 16 x 16 tiles when that gives at least twice the workgroups.
    // Larger outputs stay on the bigger tiles, which re-read the operands
    // less.
    const int64_t tiny_wgs = batch * (m / 16) * (n / 16);
    const bool tiny_ok = !d.has_cs && m % 16 == 0 && n % 16 == 0 && k % 256 == 0 && k <= 1024 &&
                         tiny_wgs <= 1024;
    if (best >= 0) {
        p.bm = cands[best].bm;
        p.bn = cands[best].bn;
        p.slice_k = cdiv(cdiv(k, best_splits), BK) * BK;
        p.splits = cdiv(k, p.slice_k);
        // Long-k products (a weight gradient Xᵀ·dY over T = 4,096 tokens):
        // slices of at most 16 k-stages, the count doubled while fewer than
        // 256 workgroups run.  Measured on MI355X (f16 route, as single calls):
        // 256x4096x768 19.0 -> 16.0 us, 256x4096x1024 18.7 -> 18.3 us,
        // 1024x4096x256 19.5 -> 18.6 us, 256x4096x256 unchanged at 16 slices;
        // the same rule on k = 768..1,024 products (split 2) was 3-5 us slower.
        if (can_split && k >= 2048) {
            const int64_t tiles = batch * (m / p.bm) * (n / p.bn);
            int64_t sp = 1;
            while (k / sp > 16 * BK && k / (2 * sp) >= 4 * BK && sp < 64) sp *= 2;
            while (tiles * sp < 256 && k / (2 * sp) >= 8 * BK) sp *= 2;
            p.slice_k = cdiv(cdiv(k, sp), BK) * BK;
            p.splits = cdiv(k, p.slice_k);
        }
    }
    const int64_t dma_wgs = best >= 0 ? batch * (m / p.bm) * (n / p.bn) * p.splits : 0;
    p.tiny = tiny_ok && (best < 0 || (dma_wgs < 256 && tiny_wgs >= 2 * dma_wgs));
    if (p.tiny) {
        p.bm = p.bn = 16;
        p.splits = 1;
        p.slice_k = k;
        return true;
    }
    if (best < 0) return false;
    return !(batch * p.splits > 65535 || m / p.bm > 65535 || n / p.bn > INT32_MAX);
}

}  // namespace

namespace st {

bool gemm_dma_takes(const DmaGemm &d) {
    DmaPlan p;
    return dma_plan(d, p);
}

size_t gemm_dma_scratch(const DmaGemm &d) {
    DmaPlan p;
    if (!dma_plan(d, p) || p.splits <= 1) return 0;
    return sizeof(float) * (size_t)(d.batch * p.splits * (d.m * d.n + (d.has_cs ? d.n : 0)));
}

bool gemm_dma(const DmaGemm &d, hipStream_t stream, st_status *status) {
    DmaPlan plan;
    if (!dma_plan(d, plan)) return false;
    const int64_t m = d.m, n = d.n, k = d.k, batch = d.batch;
    const int bm = plan.bm, bn = plan.bn;
    const int64_t slice_k = plan.slice_k, splits = plan.splits;

    KArgs g;
    std::memset(&g, 0, sizeof g);
    g.a = d.a;
    g.a_stride = d.a_stride;
    g.a_group = d.a_group;
    g.a_inner = d.a_inner;
    g.lda = d.lda;
    g.b = d.b;
    g.b_stride = d.b_stride;
    g.b_group = d.b_group;
    g.b_inner = d.b_inner;
    g.ldb = d.ldb;
    g.out = d.out;
    g.o_stride = d.o_stride;
    g.o_group = d.o_group;
    g.o_inner = d.o_inner;
    g.ldo = d.ldo;
    g.bias = d.bias;
    g.bias_stride = d.bias_stride;
    g.mask = d.mask;
    g.res = d.res;
    g.cs = d.cs;
    g.cs_stride = d.cs_stride;
    g.has_cs = d.has_cs;
    g.relu = d.relu;
    g.accumulate = d.accumulate;
    g.m = (int32_t)m;
    g.n = (int32_t)n;
    g.k = (int32_t)k;
    g.splits = (int32_t)splits;
    g.slice_k = (int32_t)slice_k;
    float *part = nullptr, *cs_part = nullptr;
    if (splits > 1) {
        const size_t pfl = (size_t)(batch * splits * m * n);
        const size_t cfl = d.has_cs ? (size_t)(batch * splits * n) : 0;
        part = static_cast<float *>(scratch(SCRATCH_SPLITK, sizeof(float) * (pfl + cfl), stream));
        if (!part) {
            *status = scratch_status();
            return true;
        }
        cs_part = part + pfl;
        g.out = part;
        g.cs = cs_part;
    }
    if (plan.tiny) {
        KernelFn tf;
        if (d.f16)
            tf = d.ta ? (d.tb ? &k_gemm_tiny<true, true, true> : &k_gemm_tiny<true, false, true>)
                      : (d.tb ? &k_gemm_tiny<false, true, true> : &k_gemm_tiny<false, false, true>);
        else
            tf = d.ta ? (d.tb ? &k_gemm_tiny<true, true, false> : &k_gemm_tiny<true, false, false>)
                      : (d.tb ? &k_gemm_tiny<false, true, false> : &k_gemm_tiny<false, false, false>);
        hipLaunchKernelGGL(tf, dim3((unsigned)(n / 16), (unsigned)(m / 16), (unsigned)batch), dim3(THREADS), 0,
                           stream, g);
        const hipError_t e = hipGetLastError();
        *status = e == hipSuccess ? ST_OK : fail(ST_ERR_HIP, "GEMM launch failed: %s", hipGetErrorString(e));
        return true;
    }
    // Ring depths: 128 KB, 96 KB, 64 KB and 8 KB per stage of 32 x 32.
    KernelFn fn;
    if (bm == 128 && bn == 128)
        fn = pick2<128, 128, 4>(d.f16, d.ta, d.tb);
    else if (bm == 128)
        fn = pick2<128, 64, 4>(d.f16, d.ta, d.tb);
    else if (bm == 64)
        fn = pick2<64, 64, 4>(d.f16, d.ta, d.tb);
    else
        fn = pick<32, 32, 4, false>(d.ta, d.tb);
    hipLaunchKernelGGL(fn, dim3((unsigned)(n / bn), (unsigned)(m / bm), (unsigned)(batch * splits)), dim3(THREADS), 0,
                       stream, g);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && splits > 1) {
        const int64_t threads = batch * (m * n / 4) + (d.has_cs ? batch * n : 0);
        hipLaunchKernelGGL(k_sum_slices, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0, stream, part, d.out, m * n,
                           (int32_t)splits, d.o_stride, batch, d.accumulate, d.has_cs ? cs_part : nullptr, d.cs,
                           d.cs_stride, n);
        e = hipGetLastError();
    }
    *status = e == hipSuccess ? ST_OK : fail(ST_ERR_HIP, "GEMM launch failed: %s", hipGetErrorString(e));
    return true;
}

}  // namespace st
