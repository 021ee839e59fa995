// Grouped GEMM: several independent GEMMs (no one reads or writes what
// another writes) in one persistent launch of the LDS-DMA tile engine
// (dma_tile.h).  The reference issues such GEMMs back to back on its queue,
// e.g. the dW and dx of a Linear backward (gpu_step/tape.rs:324-347); each
// launch of its own pays the launch, the ramp of the first k-stages and the
// drain of the last tile, which at the d_model-256 step shapes (0.5-2 GFLOP
// per GEMM) cost as much as the arithmetic.  Here every output tile (256 x 128,
// or 128 x 128 for GEMMs whose m is not a multiple of 256) or split-k slice of
// every GEMM of the group is a unit of work; one workgroup per CU walks its
// units and starts the DMA of the next unit's first k-stages while it
// multiplies the last stages of the current one, so the ring of stages never
// drains between tiles.
//
// Units are dealt to the 8 XCDs (a workgroup's XCD is its id mod 8) as one
// contiguous block of each GEMM's tiles per XCD, so the tiles an XCD runs
// together share operand panels in its L2; GEMMs are ordered by k-stages per
// unit, longest first, and each XCD's workgroups take its units round-robin.
//
// Per element the arithmetic is that of gemm_dma.hip (the same k-stage order
// and matrix-core instructions), so a GEMM that is not split here gives the
// bits of the single-GEMM kernel when that one does not split either.  Split-k
// (free epilogue but +=, packed out) writes per-slice partials that
// k_sum_group adds in ascending slice order with accumulate and the column
// sums, as k_sum_slices does (matmul.rs:259-299).
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <numeric>
#include <queue>
#include <utility>
#include <vector>

#include "dma_tile.h"
#include "lanes.h"
#include "gemm_dma.h"

namespace {

using namespace dma;

constexpr int XCDS = 8;
constexpr int TN = 128;  // output tile columns (both shapes)

// Tile shapes: TM x 128 output tiles, WGM x 2 waves of 64 x 64 each, NS
// k-stages of 32 resident in LDS.  256-row tiles (8 waves, 144 KB) read 25 %
// fewer operand bytes per flop and keep two waves per SIMD, so one wave's
// LDS reads and conversions overlap the other's matrix-core work; 128-row
// tiles (4 waves, 128 KB) serve GEMMs whose m is not a multiple of 256.
template <int TM_, int WGM_, int NS_>
struct Cfg {
    static constexpr int TM = TM_, WGM = WGM_, WGN = 2, NS = NS_;
    static constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
    static constexpr int WM = TM / WGM, WN = TN / WGN, FM = WM / 16, FN = WN / 16;
    static constexpr int SA = TM * BK, SB = TN * BK;           // floats per stage
    static constexpr int LA = TM / (8 * WAVES), LB = TN / (8 * WAVES);  // DMA wave-loads per wave per stage
    static_assert(WM == 64 && WN == 64, "64 x 64 per wave");
    static_assert(NS * (SA + SB) * 4 <= 160 * 1024, "LDS");
    // Split-k keeps a 256-row unit to half a CU's fair share of k-stages.
    // Timed on the d_model-256 training step's 15 GEMMs (fair share 39
    // stages), whose five dW GEMMs (k = 4096) the whole share cuts into 4
    // slices of 32 stages: 8 slices of 16 take the call 211.5 -> 197.1 us;
    // 16 slices of 8 220.9 us.
    static constexpr double FAIR_PART = TM == 256 ? 0.5 : 1.0;
};
using Tall = Cfg<256, 4, 3>;
using Square = Cfg<128, 2, 4>;

enum { F_TA = 1, F_TB = 2, F_RELU = 4, F_ACC = 8, F_CS = 16 };

struct GProb {
    const float *a, *b;
    float *out;  // the output, or this GEMM's split partials [batch][splits][m][n]
    const float *bias, *mask, *res;
    float *cs;  // column-sum destination (out buffer + col_sum_off), or the split partials [batch][splits][n]
    int64_t a_stride, a_inner, b_stride, b_inner, o_stride, o_inner, bias_stride, cs_stride;
    int32_t a_group, b_group, o_group;
    int32_t lda, ldb, ldo;
    int32_t m, n, k, splits, slice_k;
    int32_t flags;
    int32_t tiles_n, tiles_m;
    int32_t units;  // tiles_n * tiles_m * batch * splits
    int32_t pad;
};

// Units per XCD list that the host-computed schedule covers.
constexpr int SCHED_MAX = 128;

struct GroupArgs {
    GProb p[st::GROUP_MAX];
    int32_t count;
    // 1: owner[x][i] is the workgroup (0 .. L-1 of XCD x's L) that runs unit i
    // of x's list; 0: round robin (workgroup w runs units w, w + L, ..).
    int32_t sched;
    // Polls of a slot counter after which a wait of the f16 kernel gives up
    // (and counts the give-up in g_waits_given_up).
    uint32_t wait_polls;
    uint8_t owner[XCDS][SCHED_MAX];
};
static_assert(sizeof(GroupArgs) <= 4000, "kernel arguments");
static_assert(sizeof(GroupArgs) % 4 == 0, "copied to LDS as 32-bit words");

// A unit of work of one workgroup: one output tile (or split slice) of one GEMM.
template <class C>
struct Unit {
    int32_t p;  // GEMM index, -1: none
    int32_t nst, row0, col0, slice;
    int64_t zb;
    bool akc, bkc;
    const char *anext, *bnext;          // operand bytes of the next stage to issue (wave-uniform)
    int64_t astep, bstep;               // bytes per stage
    uint32_t aoff[C::LA], boff[C::LB];  // this lane's DMA source offsets, less the instruction offsets
};

template <int ROWS>
__device__ __forceinline__ int64_t slot_src_rt(bool kc, int p, int64_t ld, int row0) {
    return kc ? slot_src<ROWS, true>(p, ld, row0) : slot_src<ROWS, false>(p, ld, row0);
}

// A wave-uniform value read from LDS, moved to scalar registers.
__device__ __forceinline__ int32_t uni(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
template <class T>
__device__ __forceinline__ T *uni(T *v) {
    return reinterpret_cast<T *>(uni(reinterpret_cast<int64_t>(v)));
}

// Device memory reached through a global-address-space pointer.  The group's
// pointers come from LDS, so the compiler cannot tell them from LDS addresses
// and would emit flat loads and stores; a flat store also counts against the
// LDS wait counter, so the next wait for an LDS read (every consumer stage
// has one) would wait until the epilogue's stores reached memory.
template <class T>
using gptr = T __attribute__((address_space(1))) *;
template <class T>
__device__ __forceinline__ gptr<T> glb(T *p) {
    return (gptr<T>)p;
}

// First unit of XCD x's block of GEMM p's units: x U / 8 of U.
__device__ __forceinline__ int block_start(int x, int units) { return (int)((int64_t)x * units / XCDS); }

// The group's arguments in LDS (copied from the kernel-argument segment once
// per workgroup: a read of it whose index is only known at run time goes to
// memory, one dependent round trip per read) and cum[p] = the position in XCD
// x's list of GEMM p's block (cum[count] = the list's length).
__device__ __forceinline__ void load_args(const GroupArgs &ga, GroupArgs &sga, int32_t *cum, int x, int tid,
                                          int nthreads) {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(&ga);
    uint32_t *dst = reinterpret_cast<uint32_t *>(&sga);
    for (int i = tid; i < (int)(sizeof(GroupArgs) / 4); i += nthreads) dst[i] = src[i];
    __syncthreads();
    if (tid < 64) {
        const int p = tid, count = sga.count;
        const int U = p < count ? sga.p[p].units : 0;
        int v = block_start(x + 1, U) - block_start(x, U);  // inclusive prefix sum over p
#pragma unroll
        for (int d = 1; d < st::GROUP_MAX; d *= 2) {
            const int w = __shfl_up(v, d, 64);
            if (p >= d) v += w;
        }
        if (p < count) cum[p + 1] = v;
        if (p == 0) cum[0] = 0;
    }
    __syncthreads();
}

// Unit j of XCD x's list (every GEMM's block of tiles for XCD x, in order):
// the GEMM is the number of blocks that end at or before j (one ballot).
template <class C>
__device__ void locate(const GroupArgs &ga, const int32_t *cum, int x, int j, int wave, int lane, Unit<C> &u) {
    const int count = ga.count;
    const bool before = lane < count && cum[lane + 1] <= j;
    const int p = __popcll(__ballot(before));
    u.p = p < count ? p : -1;
    if (u.p < 0) return;
    const GProb &g = ga.p[p];
    const int tiles_n = uni(g.tiles_n), tiles_m = uni(g.tiles_m), splits = uni(g.splits), slice_k = uni(g.slice_k);
    const int flags = uni(g.flags), lda = uni(g.lda), ldb = uni(g.ldb);
    const int t = block_start(x, uni(g.units)) + j - uni(cum[p]);
    const int bx = t % tiles_n;
    const int r = t / tiles_n;
    const int by = r % tiles_m;
    const int zs = r / tiles_m;
    u.zb = zs / splits;
    u.slice = zs % splits;
    u.row0 = by * C::TM;
    u.col0 = bx * TN;
    const int kbeg = u.slice * slice_k;
    u.nst = (min(uni(g.k), kbeg + slice_k) - kbeg) / BK;
    u.akc = !(flags & F_TA);
    u.bkc = (flags & F_TB) != 0;
    u.anext = uni(reinterpret_cast<const char *>(g.a + zoff(u.zb, g.a_group, g.a_stride, g.a_inner) +
                                                 (u.akc ? kbeg : (int64_t)kbeg * lda)));
    u.bnext = uni(reinterpret_cast<const char *>(g.b + zoff(u.zb, g.b_group, g.b_stride, g.b_inner) +
                                                 (u.bkc ? kbeg : (int64_t)kbeg * ldb)));
    // Wave-load i of this wave fills LDS 1024 i bytes after the wave's first;
    // its sources lie at least 1024 i bytes past the base (rows >= 8 i apart
    // at ld >= 32, or k-lines >= i apart at ld >= 256; the leading dimensions
    // are checked on the host), so the offsets stay non-negative.
#pragma unroll
    for (int i = 0; i < C::LA; i++)
        u.aoff[i] = (uint32_t)(4 * slot_src_rt<C::TM>(u.akc, (wave * C::LA + i) * 64 + lane, lda, u.row0) - 1024 * i);
#pragma unroll
    for (int i = 0; i < C::LB; i++)
        u.boff[i] = (uint32_t)(4 * slot_src_rt<TN>(u.bkc, (wave * C::LB + i) * 64 + lane, ldb, u.col0) - 1024 * i);
    u.astep = 4 * (u.akc ? BK : (int64_t)BK * lda);
    u.bstep = 4 * (u.bkc ? BK : (int64_t)BK * ldb);
}

// grid: a multiple of 8 workgroups, at most one per CU (the ring takes most
// of the LDS).  Every GEMM's unit has at least NS - 1 k-stages.
template <class C>
__global__ __launch_bounds__(C::THREADS) void k_gemm_group(GroupArgs ga) {
    constexpr int TM = C::TM, NS = C::NS, SA = C::SA, SB = C::SB, LA = C::LA, LB = C::LB;
    constexpr int WM = C::WM, WN = C::WN, FM = C::FM, FN = C::FN;
    __shared__ __attribute__((aligned(16))) float lds[NS * (SA + SB)];
    __shared__ GroupArgs sga;
    __shared__ int32_t cum[st::GROUP_MAX + 1];
    static_assert(NS * (SA + SB) * 4 + sizeof(GroupArgs) + 4 * (st::GROUP_MAX + 1) <= 160 * 1024, "LDS");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::WGN, wn = wave % C::WGN;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int x = blockIdx.x % XCDS, L = gridDim.x / XCDS;
    const int w = blockIdx.x / XCDS;
    load_args(ga, sga, cum, x, tid, C::THREADS);

    // Position in x's list of this workgroup's first unit after position
    // `prev` (prev = -1: its first), or the list's length if none is left.
    const int nlist = uni(cum[sga.count]), sched = uni(sga.sched);
    auto next_pos = [&](int prev) -> int {
        if (!sched) return min(prev < 0 ? w : prev + L, nlist);
        for (int base = prev + 1; base < nlist; base += 64) {
            const int i = base + lane;
            const uint64_t mine = __ballot(i < nlist && sga.owner[x][i] == w);
            if (mine) return base + __builtin_ctzll(mine);
        }
        return nlist;
    };
    int j = next_pos(-1), jn = next_pos(j);

    Unit<C> cur, nxt;
    locate(sga, cum, x, j, wave, lane, cur);
    if (cur.p < 0) return;
    locate(sga, cum, x, jn, wave, lane, nxt);

    // The ring advances one slot per stage: islot is the byte offset of the
    // slot the next issued stage fills, rslot of the next stage to land.
    constexpr uint32_t SLOT = (SA + SB) * 4;
    const uint32_t lds0 = lds_addr_of(lds);
    uint32_t islot = 0, rslot = 0;
    auto issue = [&](Unit<C> &u) {
        const uint32_t m0a = lds0 + islot + wave_u * LA * 1024;
        dma_stage<LA, LB>(u.anext, u.aoff, m0a, u.bnext, u.boff, lds0 + islot + SA * 4 + wave_u * LB * 1024);
        u.anext += u.astep;
        u.bnext += u.bstep;
        islot = islot + SLOT == NS * SLOT ? 0 : islot + SLOT;
    };
#pragma unroll
    for (int st = 0; st < NS - 1; st++) issue(cur);

    f32x4 acc[FM][FN];  // 16 x 16 blocks (v_mfma_f32_16x16x4_f32)
    while (true) {
        const GProb &g = sga.p[cur.p];
        const int gflags = uni(g.flags), gsplits = uni(g.splits);
        const bool do_cs = (gflags & F_CS) && cur.row0 == 0;
        float cs_acc = 0.f;  // column sum of B for column col0 + tid (tid < TN), this slice
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int jn = 0; jn < FN; jn++) acc[i][jn] = f32x4{0.f, 0.f, 0.f, 0.f};

        // Stage st of cur: wait for this wave's DMA of it (younger stages,
        // possibly the next unit's, stay in flight), barrier (every wave's
        // part landed, every wave done with the previous stage), start the
        // stage NS - 1 ahead (of cur, or of nxt once cur's run out) into the
        // slot just freed, multiply.
        auto kloop = [&](auto akc_c, auto bkc_c) {
            constexpr bool AKC = decltype(akc_c)::value, BKC = decltype(bkc_c)::value;
            const int nst = cur.nst;
            const bool more = nxt.p >= 0;
            for (int st = 0; st < nst; st++) {
                const int issued = more ? st + NS - 1 : min(st + NS - 1, nst);
                wait_stage<LA + LB, NS - 2>(issued - st - 1);
                bar();
                if (st + NS - 1 < nst)
                    issue(cur);
                else if (more)
                    issue(nxt);
                const float *la = lds + rslot / 4;
                rslot = rslot + SLOT == NS * SLOT ? 0 : rslot + SLOT;
                const float *lb = la + SA;
                const int gq = lane >> 4;
                // Lane group gq supplies k = 8 gq + u at MFMA step u, for A and B alike.
                float ax[FM][8], bx8[FN][8];
#pragma unroll
                for (int i = 0; i < FM; i++) frag<TM, AKC>(la, wm * WM + i * 16 + (lane & 15), gq, ax[i]);
#pragma unroll
                for (int jn = 0; jn < FN; jn++) frag<TN, BKC>(lb, wn * WN + jn * 16 + (lane & 15), gq, bx8[jn]);
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < FM; i++)
#pragma unroll
                        for (int jn = 0; jn < FN; jn++)
                            acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x4f32(ax[i][u], bx8[jn][u], acc[i][jn], 0, 0, 0);
                if (do_cs && tid < TN) {
                    float v[8];
#pragma unroll
                    for (int gg = 0; gg < 4; gg++) {
                        frag<TN, BKC>(lb, tid, gg, v);
#pragma unroll
                        for (int e = 0; e < 8; e++) cs_acc += v[e];
                    }
                }
            }
        };
        if (cur.akc) {
            if (cur.bkc)
                kloop(std::true_type(), std::true_type());
            else
                kloop(std::true_type(), std::false_type());
        } else {
            if (cur.bkc)
                kloop(std::false_type(), std::true_type());
            else
                kloop(std::false_type(), std::false_type());
        }

        if (do_cs && tid < TN) {
            if (gsplits > 1)
                glb(g.cs)[(cur.zb * gsplits + cur.slice) * (int64_t)g.n + cur.col0 + tid] = cs_acc;
            else
                glb(g.cs)[cur.zb * g.cs_stride + cur.col0 + tid] += cs_acc;
        }
        // Epilogue through LDS: the slot of the unit's last stage is free
        // until the next unit's first barrier (the next stage issued into it
        // follows that barrier); once every wave is done reading it, each
        // wave turns its 64 x 64 accumulators into 16-byte runs of rows, 16
        // rows at a time (pitch EP: the 16 lanes of a row write 16 consecutive
        // words and its 4 row groups land 16 banks apart), and stores them
        // with the epilogue in the reference's order: + bias, ReLU, zero where
        // mask <= 0, + residual, + out.
        bar();
        {
            // Pitch: 16 banks between the 4-row groups of a 16 x 16 block.
            constexpr int EP = WN + 4;
            float *ep = lds + (rslot == 0 ? NS * SLOT : rslot) / 4 - (SA + SB) + wave * 16 * EP;
            const bool split = gsplits > 1;
            float *const P = split ? g.out + (cur.zb * gsplits + cur.slice) * (int64_t)g.m * g.n : nullptr;
            const int64_t o0 = uni(split ? 0 : zoff(cur.zb, g.o_group, g.o_stride, g.o_inner));
            const int64_t ld = uni((int64_t)(split ? g.n : g.ldo));
            const gptr<float> obase = glb(uni(split ? P : g.out + o0));
            const gptr<const float> bias = glb(uni(g.bias)), mask = glb(uni(g.mask)), res = glb(uni(g.res));
#pragma unroll
            for (int i = 0; i < FM; i++) {
#pragma unroll
                for (int jn = 0; jn < FN; jn++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        ep[(4 * (lane >> 4) + r) * EP + jn * 16 + (lane & 15)] = acc[i][jn][r];
#pragma unroll
                for (int q = 0; q < 16 * WN / 4 / 64; q++) {
                    const int e = q * 64 + lane, row = e / (WN / 4), c4 = (e % (WN / 4)) * 4;
                    f32x4 v = *reinterpret_cast<const f32x4 *>(ep + row * EP + c4);
                    const int grow = cur.row0 + wm * WM + i * 16 + row, gcol = cur.col0 + wn * WN + c4;
                    const int64_t idx = (int64_t)grow * ld + gcol;
                    if (!split) {
                        if (bias) {
                            const gptr<const float> bp = bias + cur.zb * g.bias_stride + gcol;
#pragma unroll
                            for (int x = 0; x < 4; x++) v[x] += bp[x];
                        }
                        if (gflags & F_RELU) {
#pragma unroll
                            for (int x = 0; x < 4; x++) v[x] = v[x] < 0.f ? 0.f : v[x];
                        }
                        if (mask) {
                            const f32x4 mk = *(gptr<const f32x4>)(mask + o0 + idx);
#pragma unroll
                            for (int x = 0; x < 4; x++)
                                if (mk[x] <= 0.f) v[x] = 0.f;
                        }
                        if (res) v += *(gptr<const f32x4>)(res + o0 + idx);
                        if (gflags & F_ACC) v += *(gptr<const f32x4>)(obase + idx);
                    }
                    *(gptr<f32x4>)(obase + idx) = v;
                }
            }
        }

        if (nxt.p < 0) break;
        cur = nxt;
        j = jn;
        jn = next_pos(j);
        locate(sga, cum, x, jn, wave, lane, nxt);
    }
}

// ---------------------------------------------------------------------------
// The f16 route: operands staged through registers and converted to f16 once.
//
// Eight waves, two per SIMD: four producers and four consumers.  The
// producers load each k-stage (32 deep) of both f32 operand panels into
// registers with buffer loads, three stages ahead; one stage before it is
// multiplied, they round it to f16 (RNE, two values per v_cvt_pk_f16_f32) and
// write it to the stage's LDS slot as 16-byte runs of 8 consecutive k of one
// row.  Every element is converted once, and LDS holds f16: the LDS writes
// and the consumers' fragment reads (one ds_read_b128 per 32 x 32 x 16
// operand) move half the bytes of an f32 stage.  Operands whose rows are
// contiguous in memory (A transposed, B not) are transposed in registers: a
// producer lane loads W consecutive rows on 8 consecutive k-lines and writes
// W runs of 8 k.  The consumers each own a (TM / 2) x 64 block of the TM x 128
// tile (v_mfma_f32_32x32x16_f16) and store it straight from the accumulators.
// A producer and a consumer share each SIMD, so one's loads, conversions and
// LDS writes overlap the other's matrix-core work.
//
// LDS layout of an operand region (rows x 32 k of f16, 64 bytes per row):
// k-group g (8 k) of row r at p(r) * 64 + 16 (g ^ s(r)), p(r) = r ^ ((r >> 2) &
// 3), s(r) = (r1 ^ r4) | (r0 ^ r3 ^ r5) << 1 (ri: bit i of r).  The fragment
// reads (32 consecutive rows x 2 k-groups), the k-contiguous writes (16 rows x
// 4 groups per wave) and the transposed writes (rows W l + w, one group) each
// touch every bank once per 16 lanes (64 banks) and per 8 lanes (32 banks).
//
// Stage q is multiplied from slot q % 3 while stage q + 1 is converted into
// slot (q + 1) % 3 and the loads of stages q + 2 and q + 3 are in flight
// (three register sets).  The roles hand slots over through two counters per
// slot in LDS instead of a workgroup barrier per stage: each producer wave
// adds 1 to full[s] once its part of a stage is written, each consumer wave
// adds 1 to empty[s] once it has read its fragments, and a wave waits only
// for the counter it needs (the consumers for full[s] to reach 4 (u + 1) for
// the u-th use of slot s, the producers for empty[s] to reach 4 u before
// writing it).  So neither role waits for the other's whole step: producers
// keep loading and converting through the consumers' epilogues, up to two
// stages ahead.
// Slot waits of k_gemm_group16 that gave up (per device; st_sync reads and
// clears it).
__device__ uint32_t g_waits_given_up;

namespace r16 {

// Waits until the LDS counter reaches target.  The wait is bounded, so that a
// wave always ends: after `polls` polls it gives up, and since the slot it
// guards may then be read half-written or overwritten while read, the
// give-up is counted in g_waits_given_up (a device-memory word, added to with
// a vector atomic), which st_sync reports as an error.  The protocol reaches
// every target; a give-up means a fault in it.
__device__ __forceinline__ void spin_until(uint32_t *p, uint32_t target, uint32_t polls) {
    for (uint32_t i = 0;; i++) {
        if (__hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
        if (i >= polls) {
            if (__lane_id() == 0) atomicAdd(&g_waits_given_up, 1u);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

constexpr int NSL = 3;  // LDS slots = producer register sets

template <int TM_>
struct Cfg {
    static constexpr int TM = TM_, THREADS = 512;
    static constexpr int WM = TM / 2, WN = 64;         // 2 x 2 consumer waves
    static constexpr int M32 = WM / 32, N32 = WN / 32;  // 32 x 32 blocks per consumer wave
    static constexpr int SA = TM * 64, SB = TN * 64;    // bytes of a stage (f16)
    static constexpr int SLOT = SA + SB;
    static constexpr int NS = 5;                        // every unit (split slice) keeps NS - 1 = 4 stages
    // Split-k keeps a unit to a CU's whole fair share of k-stages: finer
    // slices of the d_model-256 step's dW GEMMs (8 instead of 4, 16 stages
    // each) take that call 57.5 -> 67.5 us, the larger split-k sum included.
    static constexpr double FAIR_PART = 1.0;
    // The kernel's LDS: NSL + 1 slots (the last for the unused conversion
    // past the final stage), their column-sum partials, the slot counters,
    // the group's arguments and their prefix sums.
    static_assert((NSL + 1) * SLOT + (NSL + 1) * 4 * TN * 4 + 2 * NSL * 4 + sizeof(GroupArgs) +
                          4 * (st::GROUP_MAX + 1) <=
                      160 * 1024,
                  "LDS");
};
using Tall16 = Cfg<256>;
using Square16 = Cfg<128>;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_off(int r, int g) {
    const int p = r ^ ((r >> 2) & 3);
    const int s = (((r >> 1) ^ (r >> 4)) & 1) | (((r ^ (r >> 3) ^ (r >> 5)) & 1) << 1);
    return (uint32_t)(p * 64 + 16 * (g ^ s));
}

// Buffer resource over [p, p + 2^31): offsets are 32-bit from the unit's
// panel base (checked on the host), no range clamping.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, 0x7fffffff, 0x00020000);
}

// How one producer lane loads an operand of R rows: 8 loads per stage of
// R / 64 dwords each.  KC (k contiguous): pair i (= i 256 + lane id) is row
// i 64 + id / 4, k-group id % 4, 32 bytes in 2 (R = 256) or 4 loads; RC:
// rows W (id % 64) .. + W - 1 on k-lines 8 (id / 64) + load index.  Load n's
// source is base + off + st step + (n >> sh) pair + (n & msk) 4 W.
struct OpRef {
    const char *base;  // panel base of the unit (its first row / column and k)
    int32_t step, pair, sh, msk;
    uint32_t off;  // this lane's byte offset within a stage
    int32_t kc;
};

struct Unit16 {
    int32_t p;  // GEMM index, -1: none
    int32_t nst, row0, col0, slice, cs;
    int64_t zb;
    OpRef a, b;
};

__device__ __forceinline__ OpRef pick(bool c, const OpRef &x, const OpRef &y) {
    OpRef o;
    o.base = c ? x.base : y.base;
    o.step = c ? x.step : y.step;
    o.pair = c ? x.pair : y.pair;
    o.sh = c ? x.sh : y.sh;
    o.msk = c ? x.msk : y.msk;
    o.off = c ? x.off : y.off;
    o.kc = c ? x.kc : y.kc;
    return o;
}

template <int R>
__device__ __forceinline__ void op_ref(OpRef &o, bool kc, const float *base, int64_t ld, int id) {
    constexpr int W = R / 64;
    o.kc = kc;
    o.base = reinterpret_cast<const char *>(base);
    if (kc) {
        o.step = 4 * BK;
        o.pair = (int32_t)(64 * ld * 4);
        o.sh = W == 4 ? 1 : 2;
        o.msk = W == 4 ? 1 : 3;
        o.off = (uint32_t)((id >> 2) * ld * 4 + 32 * (id & 3));
    } else {
        o.step = (int32_t)(BK * ld * 4);
        o.pair = (int32_t)(ld * 4);
        o.sh = 0;
        o.msk = 0;
        o.off = (uint32_t)(8 * (id >> 6) * ld * 4 + 4 * W * (id & 63));
    }
}

// The 8 loads of stage st of an operand of R rows.
template <int R>
using OpRegs = typename std::conditional<R == 256, u32x4, u32x2>::type;

template <int R>
__device__ __forceinline__ void load_op(OpRegs<R> (&v)[8], const OpRef &o, int st) {
    constexpr int W = R / 64;
    const int32_t s0 = st * o.step;
    const __amdgpu_buffer_rsrc_t r = rsrc(o.base);
#pragma unroll
    for (int n = 0; n < 8; n++) {
        // KC: load n is part n & msk (4 W bytes wide) of pair n >> sh; RC:
        // k-line n (sh = msk = 0).
        const int32_t so = s0 + (n >> o.sh) * o.pair + (n & o.msk) * (4 * W);
        if constexpr (R == 256)
            v[n] = __builtin_amdgcn_raw_buffer_load_b128(r, o.off, so, 0);
        else
            v[n] = __builtin_amdgcn_raw_buffer_load_b64(r, o.off, so, 0);
    }
}

__device__ __forceinline__ float f_(uint32_t u) { return __builtin_bit_cast(float, u); }

__device__ __forceinline__ half8 cvt8(float x0, float x1, float x2, float x3, float x4, float x5, float x6,
                                       float x7) {
    half8 h;
    h[0] = (_Float16)x0;
    h[1] = (_Float16)x1;
    h[2] = (_Float16)x2;
    h[3] = (_Float16)x3;
    h[4] = (_Float16)x4;
    h[5] = (_Float16)x5;
    h[6] = (_Float16)x6;
    h[7] = (_Float16)x7;
    return h;
}

// Rounds a loaded stage of an operand of R rows to f16 and writes it to its
// LDS region.
template <int R>
__device__ __forceinline__ void store_op(const OpRegs<R> (&v)[8], bool kc, char *region, int id) {
    constexpr int W = R / 64;
    if (kc) {
        const uint32_t a = lds_off(id >> 2, id & 3);
#pragma unroll
        for (int i = 0; i < R / 64; i++) {
            half8 h;
            if constexpr (W == 4)
                h = cvt8(f_(v[2 * i][0]), f_(v[2 * i][1]), f_(v[2 * i][2]), f_(v[2 * i][3]), f_(v[2 * i + 1][0]),
                         f_(v[2 * i + 1][1]), f_(v[2 * i + 1][2]), f_(v[2 * i + 1][3]));
            else
                h = cvt8(f_(v[4 * i][0]), f_(v[4 * i][1]), f_(v[4 * i + 1][0]), f_(v[4 * i + 1][1]),
                         f_(v[4 * i + 2][0]), f_(v[4 * i + 2][1]), f_(v[4 * i + 3][0]), f_(v[4 * i + 3][1]));
            *reinterpret_cast<half8 *>(region + a + i * 4096) = h;
        }
    } else {
        const int rg = id & 63, g = id >> 6;
#pragma unroll
        for (int w = 0; w < W; w++)
            *reinterpret_cast<half8 *>(region + lds_off(W * rg + w, g)) =
                cvt8(f_(v[0][w]), f_(v[1][w]), f_(v[2][w]), f_(v[3][w]), f_(v[4][w]), f_(v[5][w]), f_(v[6][w]),
                     f_(v[7][w]));
    }
}

// The B operand (TN = 128 rows: columns of B) moves in 16-byte loads, four
// per lane and stage, so that a stage of both operands is 12 load
// instructions per producer lane instead of 16 (every load instruction costs
// the texture addresser about the same whatever its width).  RC (rows of B
// contiguous, i.e. B not transposed): lane id holds columns 4 (id % 32) .. + 3
// on k-lines 4 (id / 32) + n, n < 4; KC: row id / 8 + 32 n, k 4 (id % 8) .. + 3.
template <int R>
__device__ __forceinline__ void op_ref_b(OpRef &o, bool kc, const float *base, int64_t ld, int id) {
    static_assert(R == TN, "the B panel");
    o.kc = kc;
    o.base = reinterpret_cast<const char *>(base);
    o.sh = 0;
    o.msk = 0;
    if (kc) {
        o.step = 4 * BK;
        o.pair = (int32_t)(32 * ld * 4);
        o.off = (uint32_t)((id >> 3) * ld * 4 + 16 * (id & 7));
    } else {
        o.step = (int32_t)(BK * ld * 4);
        o.pair = (int32_t)(ld * 4);
        o.off = (uint32_t)(4 * (id >> 5) * ld * 4 + 16 * (id & 31));
    }
}

__device__ __forceinline__ void load_b(u32x4 (&v)[4], const OpRef &o, int st) {
    const int32_t s0 = st * o.step;
    const __amdgpu_buffer_rsrc_t r = rsrc(o.base);
#pragma unroll
    for (int n = 0; n < 4; n++) v[n] = __builtin_amdgcn_raw_buffer_load_b128(r, o.off, s0 + n * o.pair, 0);
}

// Rounds a loaded stage of B to f16 and writes it to its LDS region: half of
// a k-group (4 k, 8 bytes) per column (RC) or row (KC) and load.
__device__ __forceinline__ void store_b(const u32x4 (&v)[4], bool kc, char *region, int id) {
    if (kc) {
        const int c8 = id & 7;
#pragma unroll
        for (int n = 0; n < 4; n++) {
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = (_Float16)f_(v[n][e]);
            *reinterpret_cast<half4 *>(region + lds_off((id >> 3) + 32 * n, c8 >> 1) + 8 * (c8 & 1)) = h;
        }
    } else {
        // Lanes l and l + 32 of a wave hold k 0-3 and k 4-7 of one k-group
        // (kq even / odd) for the same four columns.  One v_permlane32_swap
        // per dword trades column e of the upper lane for column e + 2 of the
        // lower one, so the lower lane writes whole 8-k groups of columns 0, 1
        // and the upper lane of columns 2, 3: 16-byte writes that each touch
        // every bank once per 16 lanes (8-byte halves of a group left every
        // half-wave on half of the banks).
        const int kq = id >> 5, cg = id & 31, up = kq & 1;
        uint32_t h[4][2];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            half4 t;
#pragma unroll
            for (int n = 0; n < 4; n++) t[n] = (_Float16)f_(v[n][e]);
            const u32x2 w = __builtin_bit_cast(u32x2, t);
            h[e][0] = w[0];
            h[e][1] = w[1];
        }
#pragma unroll
        for (int e = 0; e < 2; e++) {
            u32x4 g;
#pragma unroll
            for (int d = 0; d < 2; d++) {
                const auto r = __builtin_amdgcn_permlane32_swap(h[e][d], h[e + 2][d], false, false);
                g[d] = r[0];
                g[2 + d] = r[1];
            }
            *reinterpret_cast<u32x4 *>(region + lds_off(4 * cg + e + 2 * up, kq >> 1)) = g;
        }
    }
}

template <class C>
__device__ __forceinline__ void locate16(const GroupArgs &ga, const int32_t *cum, int x, int j, int lane, int id, Unit16 &u) {
    const int count = ga.count;
    const bool before = lane < count && cum[lane + 1] <= j;
    const int p = __popcll(__ballot(before));
    u.p = p < count ? p : -1;
    if (u.p < 0) return;
    const GProb &g = ga.p[p];
    const int tiles_n = uni(g.tiles_n), tiles_m = uni(g.tiles_m), splits = uni(g.splits), slice_k = uni(g.slice_k);
    const int flags = uni(g.flags), lda = uni(g.lda), ldb = uni(g.ldb);
    const int t = block_start(x, uni(g.units)) + j - uni(cum[p]);
    const int bx = t % tiles_n;
    const int r = t / tiles_n;
    const int by = r % tiles_m;
    const int zs = r / tiles_m;
    u.zb = zs / splits;
    u.slice = zs % splits;
    u.row0 = by * C::TM;
    u.col0 = bx * TN;
    const int kbeg = u.slice * slice_k;
    u.nst = (min(uni(g.k), kbeg + slice_k) - kbeg) / BK;
    u.cs = (flags & F_CS) && u.row0 == 0;
    const bool akc = !(flags & F_TA), bkc = (flags & F_TB) != 0;
    const float *a = uni(g.a + zoff(u.zb, g.a_group, g.a_stride, g.a_inner) +
                         (akc ? (int64_t)u.row0 * lda + kbeg : (int64_t)kbeg * lda + u.row0));
    const float *b = uni(g.b + zoff(u.zb, g.b_group, g.b_stride, g.b_inner) +
                         (bkc ? (int64_t)u.col0 * ldb + kbeg : (int64_t)kbeg * ldb + u.col0));
    op_ref<C::TM>(u.a, akc, a, lda, id);
    op_ref_b<TN>(u.b, bkc, b, ldb, id);
}

// grid: a multiple of 8 workgroups, at most one per CU.  Every unit has at
// least 4 k-stages (so the loads, at most 3 stages ahead, never reach past
// the next unit).
template <class C>
__global__ __launch_bounds__(C::THREADS) void k_gemm_group16(GroupArgs ga) {
    constexpr int TM = C::TM, SA = C::SA, SLOT = C::SLOT;
    constexpr int WM = C::WM, M32 = C::M32, N32 = C::N32;
    __shared__ __attribute__((aligned(16))) char lds[(NSL + 1) * SLOT];  // + a slot for the last, unused conversion
    __shared__ float csp[NSL + 1][4][TN];  // column-sum partials of B per stage slot and k-group
    __shared__ uint32_t s_full[NSL], s_empty[NSL];
    __shared__ GroupArgs sga;
    __shared__ int32_t cum[st::GROUP_MAX + 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool producer = __builtin_amdgcn_readfirstlane(wave) >= 4;
    const int id = tid & 255;  // lane id within the producers (or the consumers)
    const int wm = (wave >> 1) & 1, wn = wave & 1;
    const int x = blockIdx.x % XCDS, L = gridDim.x / XCDS;
    const int w = blockIdx.x / XCDS;
    if (tid < NSL) {
        s_full[tid] = 0;
        s_empty[tid] = 0;
    }
    load_args(ga, sga, cum, x, tid, C::THREADS);

    const int nlist = uni(cum[sga.count]), sched = uni(sga.sched);
    const uint32_t polls = (uint32_t)uni((int32_t)sga.wait_polls);
    auto next_pos = [&](int prev) __attribute__((always_inline)) -> int {
        if (!sched) return min(prev < 0 ? w : prev + L, nlist);
        for (int base = prev + 1; base < nlist; base += 64) {
            const int i = base + lane;
            const uint64_t mine = __ballot(i < nlist && sga.owner[x][i] == w);
            if (mine) return base + __builtin_ctzll(mine);
        }
        return nlist;
    };
    int j = next_pos(-1), jn = next_pos(j);
    Unit16 cur, nxt;
    locate16<C>(sga, cum, x, j, lane, id, cur);
    if (cur.p < 0) return;
    locate16<C>(sga, cum, x, jn, lane, id, nxt);

    int st = 0;  // stage of cur being multiplied

    // ---- producer state: NSL register sets --------------------------------
    OpRegs<TM> va[NSL][8];
    u32x4 vb[NSL][4];
    // The load cursor: the unit the next loads come from (its operand
    // references by value, lu = 0 cur, 1 nxt) and its stage.  Kept apart from
    // cur / nxt so that the lane offsets the loads use change only when the
    // cursor enters a new unit.
    OpRef la = cur.a, lb = cur.b;
    int lst = 0, lnst = cur.nst, lu = 0;
    bool lvalid = true;
    // Loads the cursor's stage into register set S.  Past the workgroup's
    // last stage the loads still go out (re-reading the last unit's first
    // stage, never multiplied), so that every step has the same 12 loads in
    // flight and the compiler's waits before each conversion count the two
    // younger stages' loads exactly.
    auto issue = [&](auto set_c) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value;
        load_op<TM>(va[S], la, lvalid ? lst : 0);
        load_b(vb[S], lb, lvalid ? lst : 0);
        if (lvalid && ++lst == lnst) {
            // The loads run at most 3 stages ahead of the multiplication and
            // every unit has 4 or more: only cur's loads can run out here.
            if (lu == 0 && nxt.p >= 0) {
                la = nxt.a;
                lb = nxt.b;
                lst = 0;
                lnst = nxt.nst;
                lu = 1;
            } else {
                lvalid = false;
            }
        }
    };
    auto convert = [&](auto set_c, int ahead) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value;
        const int s = st + ahead;
        const bool in_cur = s < cur.nst, none = !in_cur && nxt.p < 0;
        // Past the last stage the dummy loads are converted too, into the
        // extra slot NSL that nobody reads: every register set is waited for
        // on every path, and no slot the consumers still read is written.
        const bool akc = in_cur || none ? cur.a.kc : nxt.a.kc, bkc = in_cur || none ? cur.b.kc : nxt.b.kc;
        const bool cs = !none && (in_cur ? cur.cs : nxt.cs);
        const int P = none ? NSL : S;
        store_op<TM>(va[S], akc, lds + P * SLOT, id);
        store_b(vb[S], bkc, lds + P * SLOT + SA, id);
        if (cs) {
            // B is row-contiguous here (the f16 route sums columns only then):
            // this lane holds columns 4 (id % 32) + e on k 4 (id / 32) .. + 3,
            // and lane id ^ 32 the other half of the k-group id / 64.  The
            // group's 8 values of a column are added in k order (the lower
            // half's sum handed up), as the single-GEMM kernel adds them.
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float p = 0.f;
#pragma unroll
                for (int n = 0; n < 4; n++) p += f_(vb[S][n][e]);
                const float lo = st::xor_lane(p, 32, lane);
                float q = lo;
#pragma unroll
                for (int n = 0; n < 4; n++) q += f_(vb[S][n][e]);
                if (lane >= 32) csp[P][id >> 6][4 * (id & 31) + e] = q;
            }
        }
    };

    // ---- consumer state ---------------------------------------------------
    // Fragment read addresses (fixed for the kernel): lane l reads row l % 32
    // of its 32-row block, k-group 2 ks + l / 32.
    uint32_t ra[M32][2], rb[N32][2];
#pragma unroll
    for (int i = 0; i < M32; i++)
#pragma unroll
        for (int ks = 0; ks < 2; ks++) ra[i][ks] = lds_off(wm * WM + i * 32 + (lane & 31), 2 * ks + (lane >> 5));
#pragma unroll
    for (int i = 0; i < N32; i++)
#pragma unroll
        for (int ks = 0; ks < 2; ks++) rb[i][ks] = SA + lds_off(wn * 64 + i * 32 + (lane & 31), 2 * ks + (lane >> 5));
    f32x16 acc[M32][N32];
#pragma unroll
    for (int i = 0; i < M32; i++)
#pragma unroll
        for (int n = 0; n < N32; n++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][n][e] = 0.f;
    float cs_acc = 0.f;  // column col0 + id of B summed over this unit's k (consumers, id < 128)

    // The epilogue of cur, straight from the accumulators: lane l holds
    // column l % 32 of each 32 x 32 block and rows 8 (e / 4) + 4 (l / 32) +
    // e % 4 of it.  The stores are nontemporal (the outputs are not read again
    // by this kernel; the step set measured ~1 % faster than with plain stores).
    auto epilogue = [&]() __attribute__((always_inline)) {
        const GProb &g = sga.p[cur.p];
        const int gflags = uni(g.flags), gsplits = uni(g.splits);
        const bool split = gsplits > 1;
        float *const P = split ? g.out + (cur.zb * gsplits + cur.slice) * (int64_t)g.m * g.n : nullptr;
        const int64_t o0 = uni(split ? 0 : zoff(cur.zb, g.o_group, g.o_stride, g.o_inner));
        const int64_t ld = uni((int64_t)(split ? g.n : g.ldo));
        const gptr<float> obase = glb(uni(split ? P : g.out + o0));
        const gptr<const float> bias = glb(uni(g.bias)), mask = glb(uni(g.mask)), res = glb(uni(g.res));
        const int64_t lane_off = (int64_t)(4 * (lane >> 5)) * ld + (lane & 31);
#pragma unroll
        for (int n = 0; n < N32; n++) {
            const int c0 = cur.col0 + wn * 64 + n * 32;
            float bv = 0.f;
            if (!split && bias) bv = bias[cur.zb * g.bias_stride + c0 + (lane & 31)];
#pragma unroll
            for (int i = 0; i < M32; i++) {
                const int64_t r0 = cur.row0 + wm * WM + i * 32;
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; e++) v[e] = acc[i][n][e];
                auto idx = [&](int e) __attribute__((always_inline)) { return (r0 + 8 * (e >> 2) + (e & 3)) * ld + c0 + lane_off; };
                if (!split) {
                    if (bias) {
#pragma unroll
                        for (int e = 0; e < 16; e++) v[e] += bv;
                    }
                    if (gflags & F_RELU) {
#pragma unroll
                        for (int e = 0; e < 16; e++) v[e] = v[e] < 0.f ? 0.f : v[e];
                    }
                    if (mask) {
                        float t[16];
#pragma unroll
                        for (int e = 0; e < 16; e++) t[e] = mask[o0 + idx(e)];
#pragma unroll
                        for (int e = 0; e < 16; e++)
                            if (t[e] <= 0.f) v[e] = 0.f;
                    }
                    if (res) {
                        float t[16];
#pragma unroll
                        for (int e = 0; e < 16; e++) t[e] = res[o0 + idx(e)];
#pragma unroll
                        for (int e = 0; e < 16; e++) v[e] += t[e];
                    }
                    if (gflags & F_ACC) {
                        float t[16];
#pragma unroll
                        for (int e = 0; e < 16; e++) t[e] = obase[idx(e)];
#pragma unroll
                        for (int e = 0; e < 16; e++) v[e] += t[e];
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; e++) __builtin_nontemporal_store(v[e], obase + idx(e));
            }
        }
        if (cur.cs && id < TN) {
            if (split)
                glb(g.cs)[(cur.zb * gsplits + cur.slice) * (int64_t)g.n + cur.col0 + id] = cs_acc;
            else
                glb(g.cs)[cur.zb * g.cs_stride + cur.col0 + id] += cs_acc;
        }
    };

    // Moves to the next unit once cur's last stage is done; false when the
    // workgroup has none left.
    auto advance = [&]() __attribute__((always_inline)) -> bool {
        if (nxt.p < 0) return false;
        cur = nxt;
        st = 0;
        lu = 0;  // the load cursor was in nxt
        j = jn;
        jn = next_pos(j);
        locate16<C>(sga, cum, x, jn, lane, id, nxt);
        return true;
    };

    // The two roles run separate loops (so their registers never live at the
    // same time), joined only by the slot counters.
    if (producer) {
        // Prologue: stages 0, 1, 2 of cur in flight; stage 0 into slot 0.
        issue(std::integral_constant<int, 0>());
        issue(std::integral_constant<int, 1>());
        issue(std::integral_constant<int, 2>());
        convert(std::integral_constant<int, 0>(), 0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes are done
        if (lane == 0) __hip_atomic_fetch_add(&s_full[0], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        uint32_t pc = 1;  // stages converted so far (over the workgroup's units)
        // Stage q (slot S): load stage q + 3 into register set S, convert
        // stage q + 1 into slot S + 1.
        auto step = [&](auto set_c) __attribute__((always_inline)) -> bool {
            constexpr int S = decltype(set_c)::value;
            // Stages q + 1 and q + 2 (12 loads each) are in flight, stage q's
            // loads are done: a no-op wait that tells the compiler so, which it
            // cannot work out through the loop's back edge by itself.
            wait_vm<24>();
            issue(set_c);
            constexpr int S1 = (S + 1) % NSL;
            const bool none = !(st + 1 < cur.nst) && nxt.p < 0;
            if (!none) spin_until(&s_empty[S1], 4 * (pc / NSL), polls);
            convert(std::integral_constant<int, S1>(), 1);
            __builtin_amdgcn_s_waitcnt(0xC07F);
            if (!none && lane == 0)
                __hip_atomic_fetch_add(&s_full[S1], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            pc++;
            return ++st < cur.nst || advance();
        };
        while (step(std::integral_constant<int, 0>()) && step(std::integral_constant<int, 1>()) &&
               step(std::integral_constant<int, 2>())) {
        }
    } else {
        uint32_t cq = 0;  // stages consumed so far
        // Stage q: multiply slot S.
        auto step = [&](auto set_c) __attribute__((always_inline)) -> bool {
            constexpr int S = decltype(set_c)::value;
            spin_until(&s_full[S], 4 * (cq / NSL + 1), polls);
            const char *slot = lds + S * SLOT;
            half8 af[2][M32], bf[2][N32];
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
#pragma unroll
                for (int i = 0; i < M32; i++) af[ks][i] = *reinterpret_cast<const half8 *>(slot + ra[i][ks]);
#pragma unroll
                for (int n = 0; n < N32; n++) bf[ks][n] = *reinterpret_cast<const half8 *>(slot + rb[n][ks]);
            }
            if (cur.cs && id < TN) {
#pragma unroll
                for (int g = 0; g < 4; g++) cs_acc += csp[S][g][id];
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);
            if (lane == 0) __hip_atomic_fetch_add(&s_empty[S], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            cq++;
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int i = 0; i < M32; i++)
#pragma unroll
                    for (int n = 0; n < N32; n++)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ks][i], bf[ks][n], acc[i][n], 0, 0, 0);
            if (++st < cur.nst) return true;
            epilogue();
#pragma unroll
            for (int i = 0; i < M32; i++)
#pragma unroll
                for (int n = 0; n < N32; n++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[i][n][e] = 0.f;
            cs_acc = 0.f;
            return advance();
        };
        while (step(std::integral_constant<int, 0>()) && step(std::integral_constant<int, 1>()) &&
               step(std::integral_constant<int, 2>())) {
        }
    }
}

}  // namespace r16

struct SProb {
    const float *part;
    float *out;
    const float *cs_part;
    float *cs_dst;
    int64_t mn4, o_stride, cs_stride, n, batch, t0;
    int32_t splits, accumulate;
};

struct SumArgs {
    SProb p[st::GROUP_MAX];
    int32_t count;
};
static_assert(sizeof(SumArgs) % 4 == 0, "copied to LDS as 32-bit words");

// The split GEMMs' partial sums, one thread per 4 outputs (then one per
// column sum), as k_sum_slices (each thread's slice loads in flight
// together); thread ranges per GEMM start at t0.  The
// arguments are copied to LDS first (as in k_gemm_group).
__global__ __launch_bounds__(256) void k_sum_group(SumArgs sa) {
    __shared__ SumArgs ssa;
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(&sa);
        uint32_t *dst = reinterpret_cast<uint32_t *>(&ssa);
        for (int i = threadIdx.x; i < (int)(sizeof(SumArgs) / 4); i += 256) dst[i] = src[i];
        __syncthreads();
    }
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int p = 0;
    while (p + 1 < ssa.count && e >= ssa.p[p + 1].t0) p++;
    const SProb &s = ssa.p[p];
    const int64_t local = e - s.t0;
    if (local < 0) return;
    if (local < s.batch * s.mn4) {
        const int64_t b = s.batch == 1 ? 0 : local / s.mn4, i = s.batch == 1 ? local : local % s.mn4;
        const gptr<const f32x4> src = (gptr<const f32x4>)s.part + b * s.splits * s.mn4 + i;
        f32x4 v = sum_slices(src, s.mn4, s.splits, f32x4{0.f, 0.f, 0.f, 0.f});
        const gptr<f32x4> o = (gptr<f32x4>)(s.out + b * s.o_stride) + i;
        if (s.accumulate) v += *o;
        *o = v;
    } else if (s.cs_part) {
        const int64_t c = local - s.batch * s.mn4;
        if (c < s.batch * s.n) {
            const int64_t b = s.batch == 1 ? 0 : c / s.n, jn = s.batch == 1 ? c : c % s.n;
            const float v = sum_slices(glb(s.cs_part) + b * s.splits * s.n + jn, s.n, s.splits, 0.f);
            glb(s.cs_dst)[b * s.cs_stride + jn] += v;
        }
    }
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool fits32(int64_t v) { return v >= 0 && v <= INT32_MAX; }

bool can_split(const st::DmaGemm &d) {
    return !d.bias && !d.relu && !d.mask && !d.res && d.ldo == d.n && d.o_group == 1 &&
           (d.batch == 1 || d.o_stride == d.m * d.n);
}

// Polls before a slot wait of k_gemm_group16 gives up (st_set_wait_limit).
constexpr uint32_t DEFAULT_WAIT_POLLS = 1u << 20;
std::atomic<uint32_t> g_wait_polls{DEFAULT_WAIT_POLLS};

}  // namespace

namespace st {

bool group_eligible(const DmaGemm &d) {
    if (d.m % Square::TM || d.n % TN || d.k % BK || d.k < 4 * BK) return false;
    if (!al16(d.a) || !al16(d.b) || !al16(d.out) || (d.mask && !al16(d.mask)) || (d.res && !al16(d.res)))
        return false;
    if (d.lda % 4 || d.ldb % 4 || d.a_stride % 4 || d.a_inner % 4 || d.b_stride % 4 || d.b_inner % 4) return false;
    if (d.ldo % 4 || d.o_stride % 4 || d.o_inner % 4) return false;
    if (d.lda < (d.ta ? d.m : d.k) || d.ldb < (d.tb ? d.k : d.n)) return false;
    if (!fits32(d.lda) || !fits32(d.ldb) || !fits32(d.ldo) || !fits32(d.a_group) || !fits32(d.b_group) ||
        !fits32(d.o_group))
        return false;
    // The f16 kernel addresses a unit's operand panels with 32-bit buffer
    // offsets below 2^31: up to 256 rows and all of k past the panel base.
    if (d.f16) {
        const auto panel_ok = [&](int64_t ld) { return (d.k + 256) * ld * 4 + 4096 < ((int64_t)1 << 31); };
        if (!panel_ok(d.lda) || !panel_ok(d.ldb)) return false;
    }
    return fits32(d.batch * (d.m / Square::TM) * (d.n / TN) * (d.k / BK));
}

bool group_tall(const DmaGemm &d) { return d.m % Tall::TM == 0; }

}  // namespace st

namespace {

// Each XCD's list of units (every GEMM's block, in kernel order) assigned to
// its L workgroups longest-processing-time first: unit by unit, in list order
// (GEMMs sorted by k-stages per unit, longest first), to the workgroup with
// the least work so far (the lowest index on ties), a unit costing its
// k-stages plus EPI_STAGES for its epilogue.  Round robin when a list is
// longer than SCHED_MAX.  Which workgroup runs a unit never changes its
// arithmetic.  The last schedule is kept per host thread with the shapes it
// was made for, so a group issued again with the same shapes reuses it.
constexpr int EPI_STAGES = 4;  // a 256 x 128 unit's epilogue: ~6-7 k cycles, ~4 stages of ~1,750

void schedule(GroupArgs &ga, int L) {
    thread_local std::vector<int32_t> last_key;
    thread_local uint8_t last_owner[XCDS][SCHED_MAX];
    thread_local int32_t last_sched = 0;
    std::vector<int32_t> key = {L, ga.count};
    for (int o = 0; o < ga.count; o++) {
        const GProb &g = ga.p[o];
        key.insert(key.end(), {g.units, g.tiles_n, g.tiles_m, g.splits, g.slice_k, g.k});
    }
    if (key == last_key) {
        ga.sched = last_sched;
        std::memcpy(ga.owner, last_owner, sizeof last_owner);
        return;
    }
    last_key.clear();  // invalid until this schedule is complete
    ga.sched = 0;
    if (L > 255) return;
    for (int x = 0; x < XCDS; x++) {
        int64_t n = 0;
        for (int o = 0; o < ga.count; o++)
            n += (int64_t)(x + 1) * ga.p[o].units / XCDS - (int64_t)x * ga.p[o].units / XCDS;
        if (n > SCHED_MAX) return;
    }
    typedef std::pair<int64_t, int> Load;  // (k-stages so far, workgroup): the smallest pops first
    for (int x = 0; x < XCDS; x++) {
        std::priority_queue<Load, std::vector<Load>, std::greater<Load>> q;
        for (int w = 0; w < L; w++) q.push(Load(0, w));
        int i = 0;
        for (int o = 0; o < ga.count; o++) {
            const GProb &g = ga.p[o];
            const int s0 = (int)((int64_t)x * g.units / XCDS), s1 = (int)((int64_t)(x + 1) * g.units / XCDS);
            for (int t = s0; t < s1; t++) {
                const int slice = (t / g.tiles_n / g.tiles_m) % g.splits;
                const int kbeg = slice * g.slice_k;
                const int nst = (std::min(g.k, kbeg + g.slice_k) - kbeg) / BK;
                Load l = q.top();
                q.pop();
                ga.owner[x][i++] = (uint8_t)l.second;
                l.first += nst + EPI_STAGES;
                q.push(l);
            }
        }
    }
    ga.sched = 1;
    last_sched = 1;
    std::memcpy(last_owner, ga.owner, sizeof last_owner);
    last_key = std::move(key);
}

// Split-k where the epilogue allows it, so that no unit holds more k-stages
// than fair_part times a CU's fair share of the whole group (taken as at
// least 8), and none fewer than 4; TM-row tiles, every slice keeps at least
// NS - 1 stages.
void group_splits(const st::DmaGemm *items, int count, int TM, int NS, double fair_part, int cus,
                  std::vector<int64_t> &splits, std::vector<int64_t> &slice_k) {
    using st::DmaGemm;
    splits.assign(count, 1);
    slice_k.assign(count, 0);
    double total = 0;
    for (int i = 0; i < count; i++)
        total += (double)items[i].batch * (items[i].m / TM) * (items[i].n / TN) * (items[i].k / BK);
    const double fair = std::max(8.0, fair_part * total / cus);
    for (int i = 0; i < count; i++) {
        const DmaGemm &d = items[i];
        int64_t sp = 1;
        if (can_split(d))
            while ((double)d.k / BK / sp > fair && d.k / (2 * sp) >= 4 * BK) sp *= 2;
        int64_t sk = cdiv(cdiv(d.k, sp), BK) * BK;
        int64_t n_sp = cdiv(d.k, sk);
        while (n_sp > 1 && d.k - (n_sp - 1) * sk < (NS - 1) * BK) {
            sp /= 2;
            sk = cdiv(cdiv(d.k, sp), BK) * BK;
            n_sp = cdiv(d.k, sk);
        }
        splits[i] = n_sp;
        slice_k[i] = sk;
    }
}

// Floats of split partials (and their column-sum partials) a grouped launch
// needs.
size_t group_part_floats(const st::DmaGemm *items, int count, const std::vector<int64_t> &splits) {
    size_t f = 0;
    for (int i = 0; i < count; i++)
        if (splits[i] > 1) {
            const st::DmaGemm &d = items[i];
            f += (size_t)(d.batch * splits[i] * d.m * d.n);
            if (d.has_cs) f += (size_t)(d.batch * splits[i] * d.n);
        }
    return f;
}

int group_cus() { return st::device_cus(); }

template <class C>
st_status launch_group(const st::DmaGemm *items, int count, void (*kern)(GroupArgs), hipStream_t stream) {
    using st::DmaGemm;
    using st::fail;
    constexpr int TM = C::TM, NS = C::NS;
    if (count <= 0) return ST_OK;
    if (count > st::GROUP_MAX) return fail(ST_ERR_INVALID, "at most %d GEMMs per grouped launch", st::GROUP_MAX);
    const int cus = group_cus();

    std::vector<int64_t> splits, slice_k;
    group_splits(items, count, TM, NS, C::FAIR_PART, cus, splits, slice_k);
    // Longest units first.
    std::vector<int> order(count);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return slice_k[x] > slice_k[y]; });

    size_t part_floats = 0;
    std::vector<size_t> part_off(count, 0), cs_off(count, 0);
    for (int i = 0; i < count; i++) {
        if (splits[i] == 1) continue;
        const DmaGemm &d = items[i];
        part_off[i] = part_floats;
        part_floats += (size_t)(d.batch * splits[i] * d.m * d.n);
        cs_off[i] = part_floats;
        if (d.has_cs) part_floats += (size_t)(d.batch * splits[i] * d.n);
    }
    float *part = nullptr;
    if (part_floats) {
        part = static_cast<float *>(st::scratch(st::SCRATCH_SPLITK, part_floats * sizeof(float), stream));
        if (!part) return st::scratch_status();
    }

    GroupArgs ga;
    std::memset(&ga, 0, sizeof ga);
    ga.wait_polls = g_wait_polls.load(std::memory_order_relaxed);
    SumArgs sa;
    std::memset(&sa, 0, sizeof sa);
    int64_t units = 0, sum_threads = 0;
    ga.count = count;
    for (int o = 0; o < count; o++) {
        const int i = order[o];
        const DmaGemm &d = items[i];
        GProb &g = ga.p[o];
        g.a = d.a;
        g.b = d.b;
        g.a_stride = d.a_stride;
        g.a_inner = d.a_inner;
        g.a_group = (int32_t)d.a_group;
        g.lda = (int32_t)d.lda;
        g.b_stride = d.b_stride;
        g.b_inner = d.b_inner;
        g.b_group = (int32_t)d.b_group;
        g.ldb = (int32_t)d.ldb;
        g.m = (int32_t)d.m;
        g.n = (int32_t)d.n;
        g.k = (int32_t)d.k;
        g.splits = (int32_t)splits[i];
        g.slice_k = (int32_t)slice_k[i];
        g.flags = (d.ta ? F_TA : 0) | (d.tb ? F_TB : 0) | (d.relu ? F_RELU : 0) | (d.accumulate ? F_ACC : 0) |
                  (d.has_cs ? F_CS : 0);
        g.tiles_n = (int32_t)(d.n / TN);
        g.tiles_m = (int32_t)(d.m / TM);
        const int64_t u = d.batch * g.tiles_n * g.tiles_m * splits[i];
        if (!fits32(u) || !fits32(units + u)) return fail(ST_ERR_INVALID, "grouped GEMM: too many tiles");
        g.units = (int32_t)u;
        units += u;
        if (splits[i] > 1) {
            // No epilogue but += and column sums, both applied by k_sum_group.
            g.out = part + part_off[i];
            g.o_stride = d.m * d.n;
            g.o_group = 1;
            g.ldo = (int32_t)d.n;
            g.cs = part + cs_off[i];
            g.cs_stride = d.n;
            g.flags &= ~F_ACC;
            SProb &s = sa.p[sa.count++];
            s.part = g.out;
            s.out = d.out;
            s.cs_part = d.has_cs ? g.cs : nullptr;
            s.cs_dst = d.cs;
            s.mn4 = d.m * d.n / 4;
            s.o_stride = d.o_stride;
            s.cs_stride = d.cs_stride;
            s.n = d.n;
            s.batch = d.batch;
            s.t0 = sum_threads;
            s.splits = (int32_t)splits[i];
            s.accumulate = d.accumulate;
            sum_threads += d.batch * s.mn4 + (d.has_cs ? d.batch * d.n : 0);
        } else {
            g.out = d.out;
            g.o_stride = d.o_stride;
            g.o_inner = d.o_inner;
            g.o_group = (int32_t)d.o_group;
            g.ldo = (int32_t)d.ldo;
            g.bias = d.bias;
            g.bias_stride = d.bias_stride;
            g.mask = d.mask;
            g.res = d.res;
            g.cs = d.cs;
            g.cs_stride = d.cs_stride;
        }
    }
    const int64_t wgs = std::min<int64_t>(cus / XCDS * XCDS, cdiv(units, XCDS) * XCDS);
    schedule(ga, (int)std::max<int64_t>(1, wgs / XCDS));
    hipLaunchKernelGGL(kern, dim3((unsigned)std::max<int64_t>(XCDS, wgs)), dim3(C::THREADS), 0, stream, ga);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && sa.count) {
        hipLaunchKernelGGL(k_sum_group, dim3((unsigned)cdiv(sum_threads, 256)), dim3(256), 0, stream, sa);
        e = hipGetLastError();
    }
    return e == hipSuccess ? ST_OK : fail(ST_ERR_HIP, "grouped GEMM launch failed: %s", hipGetErrorString(e));
}

}  // namespace

namespace st {

st_status check_group_waits() {
    constexpr int MAX_DEVICES = 64;
    static std::mutex mu;
    static void *word[MAX_DEVICES];  // device address of g_waits_given_up per device
    int dev = 0;
    ST_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return ST_OK;
    void *p = nullptr;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!word[dev]) {
            const hipError_t e = hipGetSymbolAddress(&word[dev], HIP_SYMBOL(g_waits_given_up));
            if (e != hipSuccess || !word[dev]) {
                (void)hipGetLastError();
                word[dev] = nullptr;
                return fail(ST_ERR_HIP, "hipGetSymbolAddress of the wait counter failed: %s", hipGetErrorString(e));
            }
        }
        p = word[dev];
    }
    uint32_t n = 0;
    ST_HIP_CHECK(hipMemcpy(&n, p, sizeof n, hipMemcpyDeviceToHost));
    if (n == 0) return ST_OK;
    const uint32_t zero = 0;
    ST_HIP_CHECK(hipMemcpy(p, &zero, sizeof zero, hipMemcpyHostToDevice));
    return fail(ST_ERR_HIP,
                "grouped GEMM: %u slot wait(s) gave up after %u polls; the outputs of the grouped f16 GEMMs run "
                "since the last st_sync are not valid",
                n, g_wait_polls.load(std::memory_order_relaxed));
}

size_t gemm_group_scratch(const DmaGemm *items, int count, bool f16, bool tall) {
    const int TM = tall ? 256 : 128, NS = f16 ? r16::Tall16::NS : (tall ? Tall::NS : Square::NS);
    const double fair_part = f16 ? r16::Tall16::FAIR_PART : (tall ? Tall::FAIR_PART : Square::FAIR_PART);
    std::vector<int64_t> splits, slice_k;
    group_splits(items, count, TM, NS, fair_part, group_cus(), splits, slice_k);
    return sizeof(float) * group_part_floats(items, count, splits);
}

st_status gemm_group(const DmaGemm *items, int count, bool f16, bool tall, hipStream_t stream) {
    if (f16)
        return tall ? launch_group<r16::Tall16>(items, count, &r16::k_gemm_group16<r16::Tall16>, stream)
                    : launch_group<r16::Square16>(items, count, &r16::k_gemm_group16<r16::Square16>, stream);
    return tall ? launch_group<Tall>(items, count, &k_gemm_group<Tall>, stream)
                : launch_group<Square>(items, count, &k_gemm_group<Square>, stream);
}

}  // namespace st

extern "C" st_status st_set_wait_limit(int64_t polls) {
    st::clear_error();
    if (polls > (int64_t)UINT32_MAX) return st::fail(ST_ERR_INVALID, "wait limit %lld too large", (long long)polls);
    g_wait_polls.store(polls < 0 ? DEFAULT_WAIT_POLLS : (uint32_t)polls, std::memory_order_relaxed);
    return ST_OK;
}
