// IVF probe selection on gfx950: each query's nprobe nearest cells.
//
// Reference: gpu_step/knn/ivf.rs:62-69 (Cent::new: the centroids and their
// squared norms), ivf.rs:473-489 (the query x centroid dots of search_ivf) and
// ivf.rs:128-161 (k_probe: dd = cnorm - 2 dot, the nprobe smallest, nearest
// first, ties to the lower cell id).
//
// Scoring contract (replaces the reference's f16 x f16 -> f32 dots, whose
// summation order no CPU can reproduce): centroids and queries are both
// quantised as the scan quantises a query, x_i = X_i 2^e with int16 X_i in
// [-16384, 16383] and a power-of-two scale per vector.  Then
//     dot = sum Q_i C_i                          (exact, int64)
//     dd  = cnorm - ldexp(dot, qe + ce + 1)      (one float64 subtraction)
// with cnorm = ldexp(sum C_i^2, 2 ce) (exact), and the cells are ranked by
// (dd, cell id).  The CPU oracle restates the same arithmetic.
//
// Digits.  The int16 values are split into two int8 digits, X = 256 Xh + Xl
// with Xl in [-128, 127] and Xh in [-64, 64].  One v_mfma_i32_32x32x32_i8
// takes A rows = 16 queries x {high, low} and B columns = 16 centroids x
// {high, low} over 32 dims, so its 32 x 32 int32 outputs are all four digit
// products of 256 query-centroid pairs, and dot = 65536 hh + 256 (hl + lh) +
// ll is assembled from two neighbouring lanes.  Both operands use one
// "MFMA-native" tile layout of 16 vectors (8 KiB): [k-step s][lane][16 bytes],
// lane l holding vector (l % 32) / 2, digit l % 2, dims 32 s + 16 (l / 32) ..
// + 15, so an operand is one ds_read_b128 per k-step.
//
// k_probe_prep turns the centroids into digit tiles, exponents and norms once
// per index.  Two launches per chunk of queries:
//   k_probe_part  grid = centroid slices (up to 12 tiles) x groups of 64
//                 queries.  The workgroup turns its 64 queries into digit
//                 tiles in LDS (as k_probe_prep would), stages its slice in
//                 LDS, and each wave
//                 scores its 16 queries against it, keeping the 12 x 4
//                 order-preserving dd keys of its lane in registers.  A
//                 per-query threshold -- the nprobe-th smallest of the 16
//                 per-lane minima, so at least nprobe keys lie at or below it
//                 and with them the slice's top nprobe -- leaves a few
//                 candidates per (query, slice), which go to a fixed slot of
//                 the scratch arena.  A slot that would overflow gets the
//                 slice's exact top nprobe instead (successive minima over the
//                 registers).
//   k_probe_merge one wave per query: the exact top nprobe by (dd, id) over
//                 its slots' candidates.
// A k_probe_part workgroup is 8 waves: two per query tile, each scoring half
// of the slice's tiles (two waves per SIMD hide each other's latencies).
// dd never leaves the chip; per query only the candidates (about nprobe per
// slice) are written and read back.
#include "common.h"
#include "lanes.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 256;                     // vector width (the scan's key width)
constexpr int TILE = 16;                   // vectors per digit tile
constexpr int TILE_BYTES = TILE * 2 * D;   // 8192
constexpr int PROBE_MAX = 16;              // ivf.rs:126
constexpr int QG = 64;                     // queries per k_probe_part workgroup (4 query tiles x 16)
constexpr int TPS = 12;                    // centroid tiles per slice, at most
constexpr int HT = TPS / 2;                // tiles per wave (two waves per query tile)
constexpr int PART_T = 512;                // k_probe_part threads
constexpr int CAPQ = 64;                   // candidate slot per (query, slice)
constexpr int64_t CAND_BUDGET = 256ll << 20;  // bytes of candidate slots per query chunk

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float wave_max(float v) {
    const int lane = st::lane_id();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, st::xor_lane(v, o, lane));
    return v;
}

// The quantisation of one vector value: X = clamp(rint(v / 2^(e - 14))) and
// its two digits.  ldexpf is exact here (|result| < 2^14).
__device__ __forceinline__ void digits_of(float v, int e, int32_t &xh, int32_t &xl, int32_t &X) {
    X = (int32_t)fminf(fmaxf(rintf(ldexpf(v, 14 - e)), -16384.f), 16383.f);
    xl = ((X + 128) & 255) - 128;
    xh = (X - xl) >> 8;
}

// One wave per vector r (rows n .. of the last tile are zero); lane L
// handles dims 4L .. 4L + 3, which sit in k-step L / 8, lane half (L % 8) / 4,
// bytes 4 (L % 4) ..: the two digit words go to lanes 32 h + 2 v (high) and
// + 1 (low) of the tile, v = r % 16.  Also writes the exponent and, when norm
// is not null (centroids), the exact squared norm.
__global__ __launch_bounds__(256) void k_probe_prep(const float *__restrict__ x, int64_t n, int8_t *__restrict__ dig,
                                                    int32_t *__restrict__ ex, double *__restrict__ norm) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t ntile = (n + TILE - 1) / TILE;
    if (r >= ntile * TILE) return;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (r < n) {
        const float4 f = reinterpret_cast<const float4 *>(x + r * D)[lane];
        v[0] = f.x;
        v[1] = f.y;
        v[2] = f.z;
        v[3] = f.w;
    }
    const float mx = wave_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    int e = 14;  // scale 2^0 for a zero vector
    if (mx > 0.f) frexpf(mx, &e);
    uint32_t hi = 0, lo = 0;
    int32_t s2 = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        int32_t xh, xl, X;
        digits_of(v[t], e, xh, xl, X);
        lo |= (uint32_t)(xl & 255) << (8 * t);
        hi |= (uint32_t)(xh & 255) << (8 * t);
        s2 += X * X;
    }
    const int vt = (int)(r % TILE);
    const int s = lane >> 3, h = (lane & 7) >> 2, b0 = 4 * (lane & 3);
    int8_t *blk = dig + (r / TILE) * TILE_BYTES + s * 1024 + b0;
    *reinterpret_cast<uint32_t *>(blk + (32 * h + 2 * vt) * 16) = hi;
    *reinterpret_cast<uint32_t *>(blk + (32 * h + 2 * vt + 1) * 16) = lo;
    if (r >= n) return;
    if (norm) {
        double t2 = (double)s2;  // partial sums are integers below 2^53: exact in any order
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) t2 += st::xor_lane(t2, o, lane);
        if (lane == 0) norm[r] = ldexp(t2, 2 * (e - 14));
    }
    if (lane == 0) ex[r] = e - 14;
}

// Order-preserving map of a float64 onto u64 (finite values; -0 < +0).
__device__ __forceinline__ uint64_t dkey(double v) {
    const uint64_t x = (uint64_t)__double_as_longlong(v);
    return (x >> 63) ? ~x : (x | (1ull << 63));
}

__device__ __forceinline__ bool lt(uint64_t ka, int32_t ia, uint64_t kb, int32_t ib) {
    return ka < kb || (ka == kb && ia < ib);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) { return st::xor_lane(v, m, st::lane_id()); }

// Wave-wide minimum of (key, id); every lane receives it.
__device__ __forceinline__ void wave_min(uint64_t &k, int32_t &i) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t ko = shfl_xor_u64(k, o);
        const int32_t io = st::xor_lane(i, o, st::lane_id());
        if (lt(ko, io, k, i)) {
            k = ko;
            i = io;
        }
    }
}

// Ascending bitonic sort of one u32 per lane across the wave.
__device__ __forceinline__ uint32_t wave_sort_u32(uint32_t x, int lane) {
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const uint32_t y = st::xor_lane(x, j, lane);
            const bool take_min = ((lane & j) == 0) == ((lane & k) == 0);
            x = take_min ? min(x, y) : max(x, y);
        }
    }
    return x;
}

// Ascending bitonic sort of one (key, id) pair per lane across the wave.
__device__ __forceinline__ void wave_sort_pair(uint64_t &k, int32_t &i, int lane) {
#pragma unroll
    for (int kk = 2; kk <= 64; kk <<= 1) {
#pragma unroll
        for (int j = kk >> 1; j > 0; j >>= 1) {
            const uint64_t ko = shfl_xor_u64(k, j);
            const int32_t io = st::xor_lane(i, j, lane);
            const bool take_min = ((lane & j) == 0) == ((lane & kk) == 0);
            if (take_min == lt(ko, io, k, i)) {
                k = ko;
                i = io;
            }
        }
    }
}

constexpr uint64_t KNONE = ~0ull;
constexpr int32_t INONE = 0x7fffffff;

// Candidates of (query, slice): the slot of query q (chunk-relative) and slice
// s keeps entry e at ck[(q CAPQ + e) S + s] (keys) and ci[..] (ids), so that a
// lane per slot reads an entry of consecutive slots with one coalesced load;
// pcnt[q S + s] counts them.
//
// grid: S * gy workgroups of 256 threads; workgroup b takes (slice, query
// group) = (idx / gy, idx % gy) with idx dealt so that the gy workgroups of a
// slice are consecutive on one XCD (workgroup ids go round robin over the 8
// XCDs), which then reads the slice's digits from HBM once.
__global__ __launch_bounds__(PART_T) void k_probe_part(const float *__restrict__ queries, int32_t nq,
                                                    const int8_t *__restrict__ cdig, const int32_t *__restrict__ cexp,
                                                    const double *__restrict__ cnorm, int32_t nlist, int32_t S,
                                                    int32_t gy, int32_t nprobe, uint64_t *__restrict__ ck,
                                                    int32_t *__restrict__ ci, int32_t *__restrict__ pcnt) {
    __shared__ v4i s_b[TPS * TILE_BYTES / 16];
    __shared__ double s_cn[TPS * TILE];
    __shared__ int32_t s_ce[TPS * TILE];
    __shared__ uint32_t s_x[2][4][64][4];  // per (half, query tile, lane, u): minima, then counts
    __shared__ v4i s_q[4 * TILE_BYTES / 16];  // the workgroup's 64 queries as 4 digit tiles
    __shared__ int32_t s_qe[QG];              // and their exponents
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int qt = w & 3, half = w >> 2;  // query tile; tiles [half HT, half HT + HT) of the slice
    const int64_t nb = (int64_t)S * gy, b = blockIdx.x;
    const int64_t idx = nb % 8 == 0 ? (b % 8) * (nb / 8) + b / 8 : b;
    const int32_t sl = (int32_t)(idx / gy), qg = (int32_t)(idx % gy);
    const int32_t ntiles = (nlist + TILE - 1) / TILE;
    const int32_t t0 = sl * TPS, nts = min(TPS, ntiles - t0);

    // The slice's digit tiles, norms and exponents into LDS, every load in flight.
    {
        const v4i *src = reinterpret_cast<const v4i *>(cdig + (int64_t)t0 * TILE_BYTES);
        const int n16 = nts * (TILE_BYTES / 16);
#pragma unroll
        for (int i = 0; i < TPS * TILE_BYTES / 16 / PART_T; i++)
            if (i * PART_T + tid < n16) s_b[i * PART_T + tid] = src[i * PART_T + tid];
        if (tid < nts * TILE) {
            const int32_t c = t0 * TILE + tid;
            s_cn[tid] = c < nlist ? cnorm[c] : 0.0;
            s_ce[tid] = c < nlist ? cexp[c] : 0;
        }
    }

    // The workgroup's 64 queries into digit tiles in LDS (k_probe_prep's
    // arithmetic and layout, wave w taking queries 8 w .. 8 w + 7, all eight
    // rows' loads in flight together; a query past nq is a zero row).  Every
    // slice's workgroup redoes this for its query group: 64 KB of f32 reads,
    // in place of a separate launch.
    {
        float4 f[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int32_t q = qg * QG + w * 8 + t;
            f[t] = q < nq ? reinterpret_cast<const float4 *>(queries + (int64_t)q * D)[lane]
                          : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const int s_ = lane >> 3, hh = (lane & 7) >> 2, b0 = 4 * (lane & 3);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int v = w * 8 + t;
            const float vv[4] = {f[t].x, f[t].y, f[t].z, f[t].w};
            const float mx = wave_max(fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3]))));
            int e = 14;  // scale 2^0 for a zero vector
            if (mx > 0.f) frexpf(mx, &e);
            uint32_t hi = 0, lo = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                int32_t xh, xl, X;
                digits_of(vv[k], e, xh, xl, X);
                lo |= (uint32_t)(xl & 255) << (8 * k);
                hi |= (uint32_t)(xh & 255) << (8 * k);
            }
            char *blk = reinterpret_cast<char *>(s_q) + (v / TILE) * TILE_BYTES + s_ * 1024 + b0;
            *reinterpret_cast<uint32_t *>(blk + (32 * hh + 2 * (v % TILE)) * 16) = hi;
            *reinterpret_cast<uint32_t *>(blk + (32 * hh + 2 * (v % TILE) + 1) * 16) = lo;
            if (lane == 0) s_qe[v] = e - 14;
        }
    }
    __syncthreads();

    // This wave's 16 queries (digit tile qt of the workgroup's): lane l holds
    // query (l % 32) / 2, digit l % 2, dims 32 s + 16 (l / 32) ..
    const int h = lane >> 5, odd = lane & 1;
    const int q16 = (lane & 31) >> 1;
    const int32_t qbase = qg * QG + qt * 16;
    const bool wact = qbase < nq;
    v4i a[8];
#pragma unroll
    for (int s = 0; s < 8; s++) a[s] = wact ? s_q[qt * (TILE_BYTES / 16) + s * 64 + lane] : v4i{0, 0, 0, 0};

    // Output layout of the 32 x 32 MFMA: lane l holds column l % 32 (centroid
    // c16 = (l % 32) / 2, digit l % 2) and rows 8 j + 4 h + i (i < 4, j < 4):
    // queries 4 j + 2 h (rows i = 0, 1: high, low digit) and 4 j + 2 h + 1
    // (i = 2, 3).  An even lane assembles the queries of blocks j = 0, 1, an
    // odd lane those of j = 2, 3; the lane's four queries u < 4 are
    // 4 (2 odd + u / 2) + 2 h + u % 2.
    const int c16 = q16;
    int qu[4], qeu[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        qu[u] = 4 * (2 * odd + u / 2) + 2 * h + (u & 1);
        qeu[u] = qbase + qu[u] < nq ? s_qe[qt * 16 + qu[u]] : 0;
    }
    // Every tile slot is scored (branch-free): a slot past the slice's tiles
    // reads stale LDS, and its centroid ids are >= nlist, so its keys are none.
    uint64_t key[HT][4];
    uint32_t mn[4] = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
    // The MFMAs of TG tiles at a time, k-step by k-step: TG independent
    // accumulator chains interleaved keep the matrix core busy (each MFMA's
    // input is TG instructions old); the group's keys are formed afterwards.
    constexpr int TG = 3;
    static_assert(HT % TG == 0, "tile groups");
#pragma unroll
    for (int g0 = 0; g0 < HT; g0 += TG) {
        v16i acc[TG];
#pragma unroll
        for (int t = 0; t < TG; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][i] = 0;
#pragma unroll
        for (int s = 0; s < 8; s++)
#pragma unroll
            for (int t = 0; t < TG; t++)
                acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], s_b[(half * HT + g0 + t) * 512 + s * 64 + lane],
                                                              acc[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < TG; t++) {
            const int k0 = g0 + t, k = half * HT + k0;
            // The even lane holds the products with the centroid's high digit,
            // the odd lane those with its low digit; each sends the other the
            // eight it needs.
            // (Selections by a mask, not by ?: on the two elements, which the
            // compiler would fold into a run-time index into acc.)
            const int32_t om = -odd;
            int32_t pch[8], pcl[8];
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const int32_t lo8 = acc[t][v], hi8 = acc[t][8 + v];
                const int32_t own = lo8 ^ ((lo8 ^ hi8) & om);
                const int32_t got = st::xor_lane(hi8 ^ ((lo8 ^ hi8) & om), 1, lane);
                pch[v] = own ^ ((own ^ got) & om);
                pcl[v] = got ^ ((own ^ got) & om);
            }
            const int32_t c = (t0 + k) * TILE + c16;
            const double cn = s_cn[k * TILE + c16];
            const int ce = s_ce[k * TILE + c16];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int o = 4 * (u / 2) + 2 * (u & 1);
                const int64_t dot = (int64_t)pch[o] * 65536 + (int64_t)(pcl[o] + pch[o + 1]) * 256 + pcl[o + 1];
                const double dd = cn - ldexp((double)dot, qeu[u] + ce + 1);
                key[k0][u] = k < nts && c < nlist ? dkey(dd) : KNONE;
                mn[u] = min(mn[u], (uint32_t)(key[k0][u] >> 32));
            }
        }
    }

    // Per query, the nprobe-th smallest of its 16 lanes' minima: for a given u
    // the 16 lanes of an (h, parity) group hold one query, one per centroid
    // position c16 (lane bits 1..4), so a bitonic sort over c16 by shuffles
    // puts the r-th smallest in the group's lane c16 = r.
#pragma unroll
    for (int u = 0; u < 4; u++) s_x[half][qt][lane][u] = mn[u];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; u++) mn[u] = min(mn[u], s_x[half ^ 1][qt][lane][u]);
    __syncthreads();
    uint32_t tau[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        uint32_t x = mn[u];
#pragma unroll
        for (int kk = 2; kk <= 16; kk <<= 1) {
#pragma unroll
            for (int j = kk >> 1; j > 0; j >>= 1) {
                const uint32_t y = st::xor_lane(x, 2 * j, lane);
                const bool take_min = ((c16 & j) == 0) == ((c16 & kk) == 0);
                x = take_min ? min(x, y) : max(x, y);
            }
        }
        // Lane 32 h + 2 (nprobe - 1) + odd's x: four uniform reads, one picked per lane.
        const int b = 2 * (nprobe - 1);
        const uint32_t t0 = st::lane_value(x, b), t1 = st::lane_value(x, b + 1), t2 = st::lane_value(x, b + 32),
                       t3 = st::lane_value(x, b + 33);
        tau[u] = h ? (odd ? t3 : t2) : (odd ? t1 : t0);
    }

    // Candidates: the keys at or below their query's threshold, written at the
    // count of the group's earlier candidates (a prefix sum over c16), from the
    // slot's start by the wave of tiles 0 .. HT - 1 and from its end by the
    // other.  The slot overflows when the two counts exceed CAPQ together.
    int cnt[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int32_t q = qbase + qu[u];
        uint32_t pm = 0;
#pragma unroll
        for (int k = 0; k < HT; k++) {
            const uint64_t kk = key[k][u];
            pm |= (uint32_t)(q < nq && kk != KNONE && (uint32_t)(kk >> 32) <= tau[u]) << k;
        }
        const int n = __popc(pm);
        // Inclusive sum over the group's c16 = 0 .. 15 (lanes 32 h + 2 c16 +
        // odd): DPP row shifts by 2, 4, 8 lanes scan the 8 positions of each
        // 16-lane row, then the second row of each half adds the first row's
        // total of its parity.
        int incl = n;
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, true);
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, true);
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xF, 0xF, true);
        {
            const int r0 = st::lane_value(incl, 14), r1 = st::lane_value(incl, 15), r2 = st::lane_value(incl, 46),
                      r3 = st::lane_value(incl, 47);
            if (lane & 16) incl += h ? (odd ? r3 : r2) : (odd ? r1 : r0);
        }
        {
            const int c0 = st::lane_value(incl, 30), c1 = st::lane_value(incl, 31), c2 = st::lane_value(incl, 62),
                      c3 = st::lane_value(incl, 63);
            cnt[u] = h ? (odd ? c3 : c2) : (odd ? c1 : c0);
        }
        int pos = incl - n;
        uint64_t *sk = ck + (int64_t)q * S * CAPQ + sl;
        int32_t *si = ci + (int64_t)q * S * CAPQ + sl;
#pragma unroll
        for (int k = 0; k < HT; k++) {
            if ((pm >> k) & 1) {
                if (pos < CAPQ) {
                    const int64_t at = (int64_t)(half ? CAPQ - 1 - pos : pos) * S;
                    sk[at] = key[k][u];
                    si[at] = (t0 + half * HT + k) * TILE + c16;
                }
                pos++;
            }
        }
        s_x[half][qt][lane][u] = (uint32_t)cnt[u];
    }
    __syncthreads();
    bool over = false;
    bool ov[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        ov[u] = cnt[u] + (int)s_x[half ^ 1][qt][lane][u] > CAPQ;
        over |= ov[u];
    }

    // A slot that overflowed gets each half's exact top nprobe instead (at the
    // slot's two ends): nprobe successive minima by (key, id) over the group's
    // registers, strictly above the last one taken (the four groups of a u at
    // once).
    if (__ballot(over)) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const bool mine = ov[u];
            if (!__ballot(mine)) continue;
            const int32_t q = qbase + qu[u];
            uint64_t *sk = ck + (int64_t)q * S * CAPQ + sl;
            int32_t *si = ci + (int64_t)q * S * CAPQ + sl;
            uint64_t lk = 0;
            int32_t li = -1;
            int found = 0;
            for (int r = 0; r < nprobe; r++) {
                uint64_t bk = KNONE;
                int32_t bi = INONE;
#pragma unroll
                for (int k = 0; k < HT; k++) {
                    const uint64_t kk = key[k][u];
                    const int32_t id = (t0 + half * HT + k) * TILE + c16;
                    if (kk != KNONE && lt(lk, li, kk, id) && lt(kk, id, bk, bi)) {
                        bk = kk;
                        bi = id;
                    }
                }
#pragma unroll
                for (int d = 2; d < 32; d <<= 1) {  // minimum over the group (lane bits 1..4)
                    const uint64_t ko = shfl_xor_u64(bk, d);
                    const int32_t io = st::xor_lane(bi, d, lane);
                    if (lt(ko, io, bk, bi)) {
                        bk = ko;
                        bi = io;
                    }
                }
                if (!(bk == KNONE && bi == INONE)) {
                    if (mine && c16 == 0) {
                        const int64_t at = (int64_t)(half ? CAPQ - 1 - r : r) * S;
                        sk[at] = bk;
                        si[at] = bi;
                    }
                    lk = bk;
                    li = bi;
                    found = r + 1;
                }
            }
            if (mine) cnt[u] = found;
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; u++) s_x[half][qt][lane][u] = (uint32_t)min(cnt[u], CAPQ);
    __syncthreads();
    // The slot's count: low 16 bits from its start, high 16 bits from its end.
    if (half == 0) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int32_t q = qbase + qu[u];
            if (c16 == 0 && q < nq)
                pcnt[(int64_t)q * S + sl] = (int32_t)(s_x[0][qt][lane][u] | (s_x[1][qt][lane][u] << 16));
        }
    }
}

// Entry e of a slot whose count word is c: the first (c & 0xffff) entries
// from the slot's start, then (c >> 16) from its end; -1 past them.
__device__ __forceinline__ int slot_entry(int32_t c, int e) {
    const int na = c & 0xffff, nb = (c >> 16) & 0xffff;
    return e < na ? e : e - na < nb ? CAPQ - 1 - (e - na) : -1;
}

__device__ __forceinline__ int slot_size(int32_t c) { return (c & 0xffff) + ((c >> 16) & 0xffff); }

// Candidates per lane held in registers by the merge: the first and last 16
// entries of its slot.  With 12 + 12, one query in ~30 of the benchmark's
// batch had a slot end past it and took the general path (twice as long, and
// the whole launch waited for it); 16 + 16 keeps the arrays in registers (at
// 20 + 20 the compiler moves them to scratch memory).
constexpr int MREG = 32;

// One wave per query (a workgroup of one wave, so the queries spread over
// every CU): probes[q][0, nprobe) by (key, id)
// ascending over the candidates of its S slots (lane l takes slots l, l + 64,
// ..).  A threshold on the high 32 bits of the keys is the nprobe-th smallest
// of the 64 lanes' minima, so at least nprobe candidates lie at or below it
// and every member of the top nprobe does; those (about nprobe) are gathered
// in LDS and sorted by the wave.  More than 64 of them (equal or near-equal
// distances) switch to nprobe successive minimum searches over all the
// candidates, which is exact for any input.
__global__ __launch_bounds__(256) void k_probe_merge(const uint64_t *__restrict__ ck, const int32_t *__restrict__ ci,
                                                     const int32_t *__restrict__ pcnt, int32_t nqc, int32_t S,
                                                     int32_t nprobe, int32_t *__restrict__ probes) {
    __shared__ uint64_t s_k[4][64];
    __shared__ int32_t s_i[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t q = (int64_t)blockIdx.x * (blockDim.x >> 6) + w;
    if (q >= nqc) return;
    const uint64_t *qk = ck + q * S * CAPQ;
    const int32_t *qi = ci + q * S * CAPQ;
    const int32_t *qc = pcnt + q * S;
    uint64_t *wk = s_k[w];
    int32_t *wi = s_i[w];

    // Gathers the candidates at or below tau (there are `total`, at most 64)
    // into the wave's LDS rows, lane `pos` onwards, then sorts them.
    auto finish = [&](uint64_t k, int32_t id, int total) {
        __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS stores are done
        __builtin_amdgcn_wave_barrier();
        k = lane < total ? wk[lane] : KNONE;
        id = lane < total ? wi[lane] : INONE;
        wave_sort_pair(k, id, lane);
        if (lane < nprobe) probes[q * nprobe + lane] = lane < total ? id : -1;
    };

    // One slot per lane with at most MREG / 2 candidates at either end (the
    // usual case): the ends' entries are loaded with the count, not after it
    // (each load one coalesced row of the slots), then selected from registers.
    const int32_t c0 = lane < S ? qc[lane] : 0;
    uint64_t kk[MREG];
    int32_t ii[MREG];
    if (S <= 64) {
#pragma unroll
        for (int e = 0; e < MREG; e++) {
            const int at = e < MREG / 2 ? e : CAPQ - 1 - (e - MREG / 2);
            kk[e] = lane < S ? qk[(int64_t)at * S + lane] : KNONE;
            ii[e] = lane < S ? qi[(int64_t)at * S + lane] : INONE;
        }
    }
    const int ca = c0 & 0xffff, cb = (c0 >> 16) & 0xffff;
    if (S <= 64 && !__ballot(ca > MREG / 2 || cb > MREG / 2)) {
#pragma unroll
        for (int e = 0; e < MREG; e++) {
            const bool valid = e < MREG / 2 ? e < ca : e - MREG / 2 < cb;
            if (!valid) {
                kk[e] = KNONE;
                ii[e] = INONE;
            }
        }
        uint32_t m = 0xffffffffu;
#pragma unroll
        for (int e = 0; e < MREG; e++) m = min(m, (uint32_t)(kk[e] >> 32));
        const uint32_t tau = st::lane_value(wave_sort_u32(m, lane), nprobe - 1);
        uint32_t pm = 0;
#pragma unroll
        for (int e = 0; e < MREG; e++) pm |= (uint32_t)(kk[e] != KNONE && (uint32_t)(kk[e] >> 32) <= tau) << e;
        const int mine = __popc(pm);
        const int incl = st::wave_incl_scan(mine);
        const int total = st::lane_value(incl, 63);
        if (total <= 64) {
            int pos = incl - mine;
#pragma unroll
            for (int e = 0; e < MREG; e++) {
                if ((pm >> e) & 1) {
                    wk[pos] = kk[e];
                    wi[pos] = ii[e];
                    pos++;
                }
            }
            finish(0, 0, total);
            return;
        }
        uint64_t lk = 0;
        int32_t li = -1;
        int32_t res = -1;
        for (int r = 0; r < nprobe; r++) {
            uint64_t bk = KNONE;
            int32_t bi = INONE;
#pragma unroll
            for (int e = 0; e < MREG; e++) {
                if (kk[e] != KNONE && lt(lk, li, kk[e], ii[e]) && lt(kk[e], ii[e], bk, bi)) {
                    bk = kk[e];
                    bi = ii[e];
                }
            }
            wave_min(bk, bi);
            if (bk == KNONE && bi == INONE) break;
            if (lane == r) res = bi;
            lk = bk;
            li = bi;
        }
        if (lane < nprobe) probes[q * nprobe + lane] = res;
        return;
    }

    // Any slot count and layout: the same selection, re-reading the slots.
    uint32_t m = 0xffffffffu;
    for (int32_t sl = lane; sl < S; sl += 64) {
        const int32_t c = qc[sl];
        for (int e = 0; e < slot_size(c); e++) m = min(m, (uint32_t)(qk[(int64_t)slot_entry(c, e) * S + sl] >> 32));
    }
    const uint32_t tau = st::lane_value(wave_sort_u32(m, lane), nprobe - 1);
    int mine = 0;
    for (int32_t sl = lane; sl < S; sl += 64) {
        const int32_t c = qc[sl];
        for (int e = 0; e < slot_size(c); e++)
            mine += (uint32_t)(qk[(int64_t)slot_entry(c, e) * S + sl] >> 32) <= tau;
    }
    const int incl = st::wave_incl_scan(mine);
    const int total = st::lane_value(incl, 63);
    if (total <= 64) {
        int pos = incl - mine;
        for (int32_t sl = lane; sl < S; sl += 64) {
            const int32_t c = qc[sl];
            for (int e = 0; e < slot_size(c); e++) {
                const int64_t at = (int64_t)slot_entry(c, e) * S + sl;
                const uint64_t kk = qk[at];
                if ((uint32_t)(kk >> 32) <= tau) {
                    wk[pos] = kk;
                    wi[pos] = qi[at];
                    pos++;
                }
            }
        }
        finish(0, 0, total);
        return;
    }
    uint64_t lk = 0;
    int32_t li = -1;
    int32_t res = -1;
    for (int r = 0; r < nprobe; r++) {
        uint64_t bk = KNONE;
        int32_t bi = INONE;
        for (int32_t sl = lane; sl < S; sl += 64) {
            const int32_t c = qc[sl];
            for (int e = 0; e < slot_size(c); e++) {
                const int64_t at = (int64_t)slot_entry(c, e) * S + sl;
                const uint64_t kk = qk[at];
                const int32_t ii = qi[at];
                if (lt(lk, li, kk, ii) && lt(kk, ii, bk, bi)) {
                    bk = kk;
                    bi = ii;
                }
            }
        }
        wave_min(bk, bi);
        if (bk == KNONE && bi == INONE) break;
        if (lane == r) res = bi;
        lk = bk;
        li = bi;
    }
    if (lane < nprobe) probes[q * nprobe + lane] = res;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

st_status launch_prep(const float *x, int64_t n, int8_t *dig, int32_t *ex, double *norm, hipStream_t s) {
    const int64_t rows = cdiv(n, TILE) * TILE;
    hipLaunchKernelGGL(k_probe_prep, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, x, n, dig, ex, norm);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

}  // namespace

extern "C" int64_t st_knn_centroid_digit_bytes(int64_t nlist, int64_t d) {
    if (nlist < 0 || d != D) return -1;
    return cdiv(nlist, TILE) * TILE_BYTES;
}

extern "C" st_status st_knn_centroids_prep(const float *centroids, int64_t nlist, int64_t d, int8_t *digits,
                                           int32_t *cexp, double *cnorm, st_stream stream) {
    st::clear_error();
    if (!centroids || !digits || !cexp || !cnorm) return st::fail(ST_ERR_INVALID, "centroids_prep: NULL buffer");
    if (d != D) return st::fail(ST_ERR_INVALID, "centroids_prep: built for d == %d (got %lld)", D, (long long)d);
    if (nlist < 1 || nlist > INT32_MAX / 2)
        return st::fail(ST_ERR_INVALID, "centroids_prep: nlist must be in 1..2^30 (got %lld)", (long long)nlist);
    if ((reinterpret_cast<uintptr_t>(centroids) & 15) != 0 || (reinterpret_cast<uintptr_t>(digits) & 15) != 0)
        return st::fail(ST_ERR_INVALID, "centroids_prep: centroids and digits must be 16-byte aligned");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    return launch_prep(centroids, nlist, digits, cexp, cnorm, st::stream_of(stream));
}

extern "C" st_status st_knn_probe(const int8_t *digits, const int32_t *cexp, const double *cnorm, int64_t nlist,
                                  const float *queries, int64_t nq, int64_t d, int64_t nprobe, int32_t *probes,
                                  st_stream stream) {
    st::clear_error();
    if (!digits || !cexp || !cnorm || !queries || !probes) return st::fail(ST_ERR_INVALID, "probe: NULL buffer");
    if (d != D) return st::fail(ST_ERR_INVALID, "probe: built for d == %d (got %lld)", D, (long long)d);
    if (nlist < 1 || nlist > INT32_MAX / 2 || nq < 0)
        return st::fail(ST_ERR_INVALID, "probe: bad nlist or nq");
    if (nprobe < 1 || nprobe > nlist || nprobe > PROBE_MAX)
        return st::fail(ST_ERR_INVALID, "probe: nprobe must be in 1..=min(nlist, %d) (got %lld)", PROBE_MAX,
                        (long long)nprobe);
    if ((reinterpret_cast<uintptr_t>(queries) & 15) != 0 || (reinterpret_cast<uintptr_t>(digits) & 15) != 0)
        return st::fail(ST_ERR_INVALID, "probe: queries and digits must be 16-byte aligned");
    if (nq == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const hipStream_t s = st::stream_of(stream);

    // Queries in chunks (multiples of 64) whose candidate slots fit CAND_BUDGET.
    const int64_t ntiles = cdiv(nlist, TILE), S = cdiv(ntiles, TPS);
    const int64_t per_q = S * CAPQ * (int64_t)(sizeof(uint64_t) + sizeof(int32_t)) + S * (int64_t)sizeof(int32_t);
    int64_t chunk = CAND_BUDGET / per_q;
    chunk = chunk < QG ? QG : chunk / QG * QG;
    if (chunk > nq) chunk = cdiv(nq, QG) * QG;
    if (S * cdiv(chunk, QG) > INT32_MAX) return st::fail(ST_ERR_INVALID, "probe: too many centroids");
    char *base = static_cast<char *>(st::scratch(st::SCRATCH_KNN, (size_t)(chunk * per_q), s));
    if (!base) return st::scratch_status();
    // [candidate keys][candidate ids][counts]
    uint64_t *ck = reinterpret_cast<uint64_t *>(base);
    int32_t *ci = reinterpret_cast<int32_t *>(ck + chunk * S * CAPQ);
    int32_t *pcnt = ci + chunk * S * CAPQ;

    for (int64_t q0 = 0; q0 < nq; q0 += chunk) {
        const int64_t nqc = nq - q0 < chunk ? nq - q0 : chunk;
        const int64_t gy = cdiv(nqc, QG);
        hipLaunchKernelGGL(k_probe_part, dim3((unsigned)(S * gy)), dim3(PART_T), 0, s, queries + q0 * D, (int32_t)nqc, digits,
                           cexp, cnorm, (int32_t)nlist, (int32_t)S, (int32_t)gy, (int32_t)nprobe, ck, ci, pcnt);
        ST_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_probe_merge, dim3((unsigned)nqc), dim3(64), 0, s, ck, ci, pcnt, (int32_t)nqc,
                           (int32_t)S, (int32_t)nprobe, probes + q0 * nprobe);
        ST_LAUNCH_CHECK();
    }
    return ST_OK;
}
