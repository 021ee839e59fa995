// 2-bit kNN memory on gfx950: device quantiser and the fused IVF search
// (exact integer 2-bit scoring + exact per-query top-k in one kernel).
//
// Reference: gpu_step/knn.rs:190-225 (tile_of: the 2-bit quantiser),
// knn.rs:628-643 (k_dequant: code u decodes to (u - 1.5) * scale),
// gpu_step/knn/ivf.rs:194-321 (k_scan, k_dots_group), ivf.rs:466-686
// (search_ivf / scan_group), knn.rs:655-715 (merge of per-part lists) and the
// finalisation (dd + |q|^2).max(0) (ivf.rs:673-684).
//
// Scoring contract (replaces the reference's f16 x f16 -> f32 cmma dots, whose
// accumulation order no CPU can reproduce): the query is quantised with a
// power-of-two scale qs = 2^(E-14) (max|q| = m 2^E, m in [0.5, 1)),
// Q_i = clamp(rint(q_i / qs), +-16384), and with c_i = 2u_i - 3 the key
// decodes to c_i * s / 2.  Then
//     dot  = sum c_i Q_i        (exact, int32)
//     c2   = sum c_i^2          (exact, int32)
//     dist = ((s*s)*0.25f)*(float)c2 - (s*qs)*(float)dot
// with every f32 operation separately rounded (contraction off), which the CPU
// oracle reproduces bit for bit.  Ranking is by (dist, key index) ascending.
//
// Search design: one 512-thread workgroup (8 wave64s) per query streams the
// concatenation of its probed cells in 64-key chunks, each wave with three
// chunks in flight (two waves per SIMD with up to 256 VGPRs each hold more
// bytes in flight than four waves with 128, and the scoring of one chunk
// hides behind the loads of the next two; four chunks per wave measured
// ~0.5 % slower on the 256-query batch, five ~0.7 %).  Scoring runs on the matrix cores: the key codes are FP4
// e2m1 operands as stored (a 2-bit code in the low bits of a nibble is u / 2),
// the query is four FP8 rows of balanced base-16 digits, and one scaled
// FP8 x FP4 MFMA per 128 dims gives the exact integer dot of 16 keys; one
// popcount per code dword gives c2.
//
// Top-k: each wave appends candidates with key64 = (ordered dist bits << 32 |
// index) below the shared threshold to its own LDS list (ballot + mbcnt, no
// atomics, no workgroup barrier in the scan); when the list holds 192 a
// wave-level bitonic sort keeps its 128 smallest, publishes its 8th smallest,
// and the threshold drops to the smaller of its 128th and the largest of the
// 8 waves' 16th smallest (either has 128 keys at or below it).  Only keys with
// at least 128 smaller keys are dropped, so the exact top-128 survives
// whatever the order; the output position of each survivor is its rank.
// A query's cells are scanned in increasing id order.  (Scanning the cells
// other queries of the batch also probe first, so that their second reads hit
// the MALL, bought nothing: on this device a MALL-resident buffer reads no
// faster than a stream from HBM.)
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "common.h"
#include "lanes.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 256;          // key width handled by the scan
constexpr int KMAX = 128;       // neighbours kept per query (knn.rs:21)
constexpr int CAPW = 256;       // LDS candidate list per wave (entries)
constexpr int PROBE_MAX = 16;   // most cells one query probes (ivf.rs:126)
constexpr uint64_t NONE = ~0ull;

__device__ __forceinline__ uint32_t fkey(float f) {
    uint32_t x = __float_as_uint(f);
    return (x & 0x80000000u) ? ~x : (x | 0x80000000u);
}

__device__ __forceinline__ float unfkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// ---------------------------------------------------------------- quantiser

// Row quantisation of tile_of (knn.rs:193-217) for one key held by one thread.
// `get(i)` yields component i; it is called twice per component.
template <typename Get>
__device__ __forceinline__ void quantize_row(Get get, int d, uint8_t *row, float *scale_out) {
    float ss = 0.f;
    for (int i = 0; i < d; i++) {
        const float x = get(i);
        ss += x * x;
    }
    float scale = 0.9957f * sqrtf(ss / (float)d);
    if (!(scale >= 1e-30f)) scale = 1e-30f;
    for (int w = 0; w < d / 16; w++) {
        uint32_t word = 0;
        for (int c = 0; c < 16; c++) {
            float u = roundf(get(16 * w + c) / scale + 1.5f);
            u = fminf(fmaxf(u, 0.f), 3.f);
            word |= ((uint32_t)u & 3u) << (2 * c);
        }
        reinterpret_cast<uint32_t *>(row)[w] = word;
    }
    *scale_out = scale;
}

__global__ __launch_bounds__(256) void k_quantize(const float *__restrict__ keys, int64_t n, int32_t d,
                                                  uint8_t *__restrict__ codes, float *__restrict__ scales) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const float *k = keys + r * d;
    quantize_row([&](int i) { return k[i]; }, d, codes + r * (d / 4), scales + r);
}

// The reference's stored per-key norm (knn.rs:216): sum over the dims, in
// order, of f16((u - 1.5) scale)^2 in f32; one thread per key.
__global__ __launch_bounds__(256) void k_key_norms(const uint8_t *__restrict__ codes, const float *__restrict__ scales,
                                                   int64_t n, int32_t d, float *__restrict__ norms) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const uint8_t *row = codes + r * (d / 4);
    const float s = scales[r];
    float nrm = 0.f;
    for (int i = 0; i < d; i++) {
        const int u = (row[i >> 2] >> (2 * (i & 3))) & 3;
        // The f32 product, then f16: the reference rounds twice.  The empty asm
        // keeps the compiler from fusing the two into one mixed-precision FMA
        // (a single rounding, which differs on f16 ties).
        float p = ((float)u - 1.5f) * s;
        asm volatile("" : "+v"(p));
        const float v = (float)(_Float16)p;
        nrm += v * v;
    }
    norms[r] = nrm;
}

// Counter-based N(0,1) generator for the synthetic store: a 64-bit mix of
// (seed, row, pair index) gives two uniforms, Box-Muller gives two normals.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x ^= x >> 30;
    x *= 0xbf58476d1ce4e5b9ull;
    x ^= x >> 27;
    x *= 0x94d049bb133111ebull;
    x ^= x >> 31;
    return x;
}

__device__ __forceinline__ float synth_gauss(uint64_t seed, int64_t row, int i) {
    const uint64_t h = mix64(seed ^ mix64((uint64_t)row * 0x9e3779b97f4a7c15ull + (uint64_t)(i >> 1)));
    const float u1 = ((float)(uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);  // (0, 1)
    const float u2 = (float)(uint32_t)(h & 0xffffffu) * (1.0f / 16777216.0f);     // [0, 1)
    const float r = sqrtf(-2.0f * logf(u1));
    float sv, cv;
    sincosf(6.2831853071795864f * u2, &sv, &cv);
    return (i & 1) ? r * sv : r * cv;
}

__global__ __launch_bounds__(256) void k_synth_store(uint64_t seed, int64_t row0, int64_t n, int32_t d,
                                                     uint8_t *__restrict__ codes, float *__restrict__ scales) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const int64_t row = row0 + t;
    quantize_row([&](int i) { return synth_gauss(seed, row, i); }, d, codes + t * (d / 4), scales + t);
}

__global__ __launch_bounds__(256) void k_synth_keys(uint64_t seed, int64_t row0, int64_t n, int32_t d,
                                                    float *__restrict__ keys) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n * d) return;
    keys[e] = synth_gauss(seed, row0 + e / d, (int)(e % d));
}

// ---------------------------------------------------------------- fused search

constexpr int SW = 8;           // waves per search workgroup
constexpr int STH = SW * 64;    // threads per search workgroup (one workgroup per query)
constexpr int NF = 3;           // chunks in flight per wave
static_assert(NF >= 3, "the scan's first phase scores two chunks while a third loads");

__device__ __forceinline__ float wave_max(float v) {
    const int lane = st::lane_id();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, st::xor_lane(v, o, lane));
    return v;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m, int lane) { return st::xor_lane(v, m, lane); }

// Bitonic networks over the 64 R keys of one wave held in registers: element
// e = 64 r + lane sits in lane `lane`, register r.  Exchanges across lanes
// (distance < 64) are shuffles, across registers (distance >= 64) swaps
// within the lane.  One pass (k, j) orders each pair (e, e ^ j) ascending when
// e & k == 0, descending otherwise.
template <int R, int K, int J>
__device__ __forceinline__ void bitonic_pass(uint64_t (&x)[R], int lane) {
    if constexpr (J >= 64) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            if ((r & (J / 64)) == 0) {
                const int p = r | (J / 64);
                const bool asc = ((r * 64) & K) == 0;
                const uint64_t a = x[r], b = x[p];
                const uint64_t lo = a < b ? a : b, hi = a < b ? b : a;
                x[r] = asc ? lo : hi;
                x[p] = asc ? hi : lo;
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint64_t y = shfl_xor_u64(x[r], J, lane);
            const bool asc = ((r * 64 + lane) & K) == 0;
            const bool take_min = ((lane & J) == 0) == asc;
            x[r] = (take_min == (x[r] < y)) ? x[r] : y;
        }
    }
}

// The passes j = J, J/2, .., 1 of stage K.
template <int R, int K, int J>
__device__ __forceinline__ void bitonic_stage(uint64_t (&x)[R], int lane) {
    bitonic_pass<R, K, J>(x, lane);
    if constexpr (J > 1) bitonic_stage<R, K, J / 2>(x, lane);
}

// Sorts the 64 R keys ascending (stages K = 2, 4, .., 64 R).
template <int R, int K = 2>
__device__ __forceinline__ void bitonic_sort(uint64_t (&x)[R], int lane) {
    bitonic_stage<R, K, K / 2>(x, lane);
    if constexpr (K < 64 * R) bitonic_sort<R, 2 * K>(x, lane);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    const int lane = st::lane_id();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t w = st::xor_lane(v, o, lane);
        v = w > v ? w : v;
    }
    return v;
}

// Query quantisation by one wave: qs = 2^(E-14) with max|q| = m 2^E,
// Q = clamp(rint(q / qs), -16384, 16383).  Lane l writes Q of dims 4l .. 4l + 3
// to sQ; every lane returns qs, |Q qs|^2 (from an exact sum of Q^2) and sum Q.
struct QInfo {
    float qs, qn;
    int32_t sq;
};

__device__ __forceinline__ QInfo quantize_query(const float *qrow, int lane, int16_t *sQ) {
    const float4 v = reinterpret_cast<const float4 *>(qrow)[lane];
    const float x[4] = {v.x, v.y, v.z, v.w};
    const float mx = wave_max(fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))));
    int e = 14;  // scale 2^0 for a zero query
    if (mx > 0.f) frexpf(mx, &e);
    const float qs = ldexpf(1.f, e - 14);
    int32_t sq = 0;
    double sq2 = 0.0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        // x / 2^(e-14), exact (|result| < 2^14) even where 2^(e-14) is subnormal
        const int32_t Q = (int32_t)fminf(fmaxf(rintf(ldexpf(x[t], 14 - e)), -16384.f), 16383.f);
        sq += Q;
        sq2 += (double)Q * (double)Q;
        sQ[4 * lane + t] = (int16_t)Q;
    }
    // Butterfly over the wave, written out so that every distance is a constant (a loop here is
    // not unrolled, and a run-time distance would take the ds_bpermute path).
    auto fold = [&](int o) __attribute__((always_inline)) {
        sq += st::xor_lane(sq, o, lane);
        sq2 += st::xor_lane(sq2, o, lane);
    };
    fold(32);
    fold(16);
    fold(8);
    fold(4);
    fold(2);
    fold(1);
    return QInfo{qs, (float)sq2 * (qs * qs), sq};
}

typedef int32_t v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Matrix-core operands.  The key side (B, 128 x 16 per k-step, FP4 e2m1): a
// code u kept in the low two bits of a nibble is the e2m1 number u / 2 (0, 0.5,
// 1, 1.5), so w & 0x33333333 and (w >> 2) & 0x33333333 are ready operands:
// nibble j of the first is code 2j of code dword w, of the second code 2j + 1.
// Lane l supplies column l % 16 (a key) and the 32 values of k-block l / 16; at
// k-step m (0, 1) they are dims 16 (4 (l/16) + 2m) + [0, 2, .., 14], then + 1,
// then the same for code dword 4 (l/16) + 2m + 1: FP4 nibble n of k-block h is
// k = 32 h + n.  The query side (A, FP8 e4m3) orders k differently: byte n of
// lane group g is k = 16 g + n for n < 16 and k = 64 + 16 g + (n - 16) above.
// Row 4s + p holds twice the balanced base-16 digit p of query slot s's Q
// (Q = d0 + 16 d1 + 256 d2 + 4096 d3, d0..d2 in [-8, 7], d3 in [-4, 4]; 2d is
// exact in FP8) at the dim its k pairs with; rows of absent slots are zero.
// Row 4s + p of the product is then the integer sum_i d_p,i u_i, exact in the
// f32 accumulator.  sQ holds nslot queries of D values each.
__device__ __forceinline__ void build_aq(const int16_t *sQ, int nslot, int row, int col, v8i (&aq)[2]) {
    const int slot = col >> 2, digit = col & 3;
    const int16_t *Qs = sQ + (slot < nslot ? slot : 0) * D;
#pragma unroll
    for (int m = 0; m < 2; m++) {
#pragma unroll
        for (int v = 0; v < 8; v++) {
            // elements 4v .. 4v + 3 of this lane's 32
            float f[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int n = 4 * v + e;
                const int k = n < 16 ? 16 * row + n : 64 + 16 * row + (n - 16);
                const int nb = k & 31;
                const int dword = 4 * (k >> 5) + 2 * m + (nb >> 4);
                const int code = 2 * (nb & 7) + ((nb >> 3) & 1);
                int32_t Q = Qs[16 * dword + code];
                int32_t dgt = 0;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int32_t d = p < 3 ? ((Q + 8) & 15) - 8 : Q;
                    if (p == digit) dgt = d;
                    Q = (Q - d) >> 4;
                }
                f[e] = slot < nslot ? (float)(2 * dgt) : 0.f;
            }
            int32_t word = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
            word = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], word, true);
            aq[m][v] = word;
        }
    }
}

// 64 consecutive keys from row `base`: lane l holds bytes 16 (l/16) .. of key
// 16G + l%16 for group G (the 16-byte key operand of matrix-core column l%16,
// k-block l/16; a wave's load reads 1 KB of consecutive codes) and the scale of
// key base + l.  Lanes lo <= l < hi carry keys of the scan; the rest are
// ignored.  A store of fewer than 64 keys (SMALL) is read from base 0 with
// each key index clamped to the store.
struct Chunk {
    uint4 c[4];
    float sc;
    int64_t base;
    int32_t lo, hi, g;
};

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// The codes are read with nontemporal (streaming) loads: a query reads each of
// its keys once, and the device sustains a higher read rate for streaming
// loads than for loads that allocate for reuse (about 6.8 against 6.0 TB/s).
// The scales keep ordinary loads (256 B per chunk; streaming them measured
// slower).
template <bool SMALL>
__device__ __forceinline__ void load_chunk(const uint8_t *codes, const float *scales, int64_t base, int64_t nrows,
                                           int row, int col, int lane, Chunk &ch) {
    const v4u *cb = reinterpret_cast<const v4u *>(codes + base * (D / 4));
#pragma unroll
    for (int G = 0; G < 4; G++) {
        int32_t kk = 16 * G + col;
        if (SMALL) kk = kk < nrows ? kk : 0;
        const v4u t = __builtin_nontemporal_load(cb + kk * 4 + row);
        ch.c[G] = uint4{t.x, t.y, t.z, t.w};
    }
    ch.sc = scales[base + (SMALL ? (lane < nrows ? lane : 0) : lane)];
}

// Scores one chunk against up to 4 query slots: lane l ends with d[s] =
// sum_i u_i Q_s,i and n12 = #{i: u_i in {1, 2}} for key base + l.
__device__ __forceinline__ void score_chunk(const Chunk &ch, const v8i (&aq)[2], int32_t (&d)[4], int32_t &n12) {
    int32_t vg[4], pc[4];
#pragma unroll
    for (int G = 0; G < 4; G++) {
        const uint32_t w[4] = {ch.c[G].x, ch.c[G].y, ch.c[G].z, ch.c[G].w};
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const v8i bk = {(int32_t)(w[2 * m] & 0x33333333u), (int32_t)((w[2 * m] >> 2) & 0x33333333u),
                            (int32_t)(w[2 * m + 1] & 0x33333333u), (int32_t)((w[2 * m + 1] >> 2) & 0x33333333u),
                            0, 0, 0, 0};
            // A: FP8 e4m3 (cbsz 0), B: FP4 e2m1 (blgp 4), unit block scales (E8M0 127).
            acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aq[m], bk, acc, 0, 4, 0, 127, 0, 127);
        }
        // Lane group s holds rows 4s .. 4s + 3 (slot s's digit sums) in
        // registers 0..3; sum u Q = sum_p 16^p (row 4s + p), every step an
        // exact integer.
        const float dq = __builtin_fmaf(16.f, __builtin_fmaf(16.f, __builtin_fmaf(16.f, acc[3], acc[2]), acc[1]),
                                        acc[0]);
        vg[G] = (int32_t)dq;
        // Codes with u in {1, 2} of key 16G + col among this lane's 64 dims.
        int32_t p = 0;
#pragma unroll
        for (int s = 0; s < 4; s++) p += __popc((w[s] ^ (w[s] >> 1)) & 0x55555555u);
        pc[G] = p;
    }
    // vg[G] in lane group s is slot s's dot of key 16G + col: transpose the
    // 4 x 4 (register, lane group) blocks so that d[s] in lane group G holds
    // it (lane l ends with key l's dots); sum group G's counts over the four
    // lane groups into lane group G.
    auto a = __builtin_amdgcn_permlane32_swap((unsigned)vg[0], (unsigned)vg[2], false, false);
    auto b = __builtin_amdgcn_permlane32_swap((unsigned)vg[1], (unsigned)vg[3], false, false);
    auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    auto e = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    d[0] = (int32_t)c[0];
    d[1] = (int32_t)c[1];
    d[2] = (int32_t)e[0];
    d[3] = (int32_t)e[1];
    auto x = __builtin_amdgcn_permlane32_swap((unsigned)pc[0], (unsigned)pc[2], false, false);
    auto y = __builtin_amdgcn_permlane32_swap((unsigned)pc[1], (unsigned)pc[3], false, false);
    auto z = __builtin_amdgcn_permlane16_swap(x[0] + x[1], y[0] + y[1], false, false);
    n12 = (int32_t)(z[0] + z[1]);
}

constexpr int E8 = (KMAX + SW - 1) / SW;  // each wave's published rank: SW * E8 >= KMAX keys

typedef __attribute__((address_space(3))) uint64_t lds_u64;

struct Kept {
    int32_t na;    // keys kept (sorted at wl[0, na))
    uint64_t tau;  // the 128th smallest kept key, NONE while fewer
};

// Merges a wave's nb new keys (wl[KMAX, KMAX + nb), nb <= 128) into its na
// kept ones (wl[0, na), sorted): the new keys are sorted in registers, the
// minimum of each kept key and the mirrored new key (a bitonic split) holds
// the 128 smallest of both, and a bitonic merge sorts them into wl[0, KMAX).
// The E8R-th smallest goes to *e8 (when there are E8R).  Not inlined: it runs a
// few times per wave and query, and inlined its registers would spill the
// scan loop's.
template <int E8R>
__device__ __attribute__((noinline)) Kept merge_new_keys(lds_u64 *wl, int na, int nb, lds_u64 *e8, int lane) {
    uint64_t nk[2], kp[2];
#pragma unroll
    for (int r = 0; r < 2; r++) nk[r] = r * 64 + lane < nb ? wl[KMAX + r * 64 + lane] : NONE;
    bitonic_sort<2>(nk, lane);
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const uint64_t a = r * 64 + lane < na ? wl[r * 64 + lane] : NONE;
        const uint64_t b = shfl_xor_u64(nk[1 - r], 63, lane);  // new key 127 - (64 r + lane)
        kp[r] = a < b ? a : b;
    }
    bitonic_stage<2, 128, 64>(kp, lane);
    wl[lane] = kp[0];
    wl[64 + lane] = kp[1];
    if (lane == E8R - 1 && kp[0] != NONE) *e8 = kp[0];
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    Kept k;
    k.na = __popcll(__ballot(kp[0] != NONE)) + __popcll(__ballot(kp[1] != NONE));
    k.tau = ((uint64_t)st::lane_value((uint32_t)(kp[1] >> 32), 63) << 32) | st::lane_value((uint32_t)kp[1], 63);
    return k;
}

// grid: one workgroup of 1024 threads per query.  IVF mode (MASKED false):
// the query scans its probed cells (probes, cell_start).  MASKED: it scans
// the keys g < always and lo <= g < hi of the store's nkeys (lohi [nq, 2]),
// as two row segments; cell_start, probes, ncells and nprobe are unused.
template <bool MASKED>
__global__ __launch_bounds__(STH) void k_search(const uint8_t *codes, const float *scales,
                                                const int64_t *__restrict__ cell_start, int64_t ncells,
                                                const float *__restrict__ queries, const int32_t *__restrict__ probes,
                                                int32_t nq, int32_t nprobe, int32_t k, int64_t *__restrict__ out_idx,
                                                float *__restrict__ out_dist, const int64_t *__restrict__ lohi,
                                                int64_t always, int64_t nkeys) {
    __shared__ uint64_t cand[SW * CAPW];  // per-wave candidate lists
    __shared__ uint64_t fin[SW * KMAX];   // the final gather
    __shared__ uint64_t s_tau;            // shared threshold (only decreases)
    __shared__ uint64_t s_e8[SW];         // each wave's E8-th smallest kept key
    __shared__ int16_t s_Q[D];
    __shared__ float s_qs, s_qn;
    __shared__ int32_t s_sq, s_np, count, s_next;
    __shared__ int64_t s_r0[PROBE_MAX], s_nrows;
    __shared__ int32_t s_len[PROBE_MAX], s_cpre[PROBE_MAX + 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t q = blockIdx.x;

    if (wave == 0) {
        const QInfo qi = quantize_query(queries + q * D, lane, s_Q);
        if (lane == 0) {
            s_qs = qi.qs;
            s_qn = qi.qn;
            s_sq = qi.sq;
        }
    } else if (wave == 1 && MASKED) {
        if (lane == 0) {
            // Segments [0, min(always, nkeys)) and [max(lo, always), min(hi, nkeys)).
            const int64_t lo = lohi[2 * q], hi = lohi[2 * q + 1];
            const int64_t a1 = always < nkeys ? always : nkeys;
            const int64_t b0 = lo > always ? lo : always, b1 = hi < nkeys ? hi : nkeys;
            int np = 0;
            s_cpre[0] = 0;
            if (a1 > 0) {
                s_r0[np] = 0;
                s_len[np] = (int32_t)a1;
                s_cpre[np + 1] = (int32_t)((a1 + 63) / 64);
                np++;
            }
            if (b1 > b0) {
                s_r0[np] = b0;
                s_len[np] = (int32_t)(b1 - b0);
                s_cpre[np + 1] = s_cpre[np] + (int32_t)((b1 - b0 + 63) / 64);
                np++;
            }
            s_np = np;
            s_nrows = nkeys;
        }
    } else if (wave == 1) {
        // The probed cells in increasing id order (lane j loads probe j; all
        // loads in flight together), a repeated id once, an id outside
        // [0, ncells) skipped; s_cpre counts 64-key chunks.  Each lane finds its
        // cell's place from the other lanes' ids (readlane), with no serial
        // sort.
        const int32_t c = lane < nprobe ? probes[q * nprobe + lane] : -1;
        const bool ok = lane < nprobe && c >= 0 && c < ncells;
        const int64_t r0 = ok ? cell_start[c] : 0, r1 = ok ? cell_start[c + 1] : 0;
        if (lane == 63) s_nrows = cell_start[ncells];
        const int32_t key = ok ? c : INT32_MAX;
        bool dup = false;
        for (int i = 0; i < nprobe; i++) dup |= i < lane && __builtin_amdgcn_readlane(key, i) == key;
        const bool keep = ok && !dup;
        const int32_t nch = keep ? (int32_t)((r1 - r0 + 63) / 64) : 0;
        int32_t pos = 0, cum = 0;
        for (int i = 0; i < nprobe; i++) {
            const int32_t ki = __builtin_amdgcn_readlane(key, i);
            const bool kpi = __builtin_amdgcn_readlane((int32_t)keep, i) != 0;
            pos += kpi && ki < key;
            cum += kpi && ki <= key ? __builtin_amdgcn_readlane(nch, i) : 0;
        }
        if (keep) {
            s_r0[pos] = r0;
            s_len[pos] = (int32_t)(r1 - r0);
            s_cpre[pos + 1] = cum;
        }
        const int np = __popcll(__ballot(keep));
        if (lane == 0) {
            s_cpre[0] = 0;
            s_np = np;
        }
    } else if (wave == 2) {
        if (lane < SW) s_e8[lane] = NONE;
        if (lane == 0) {
            s_tau = NONE;
            count = 0;
            s_next = 0;
        }
    }
    __syncthreads();

    const int row = lane >> 4, col = lane & 15;
    v8i aq[2];
    build_aq(s_Q, 1, row, col, aq);
    const float qs = s_qs;
    const int32_t sq = s_sq;
    const int np = s_np;
    const int32_t nchunks = s_cpre[np];
    const int64_t nrows = s_nrows;
    const int32_t c2_base = 9 * D;

    // The waves take chunks of the query's cells (taken in order) from a
    // shared counter, so each wave's chunks come in increasing order and a fast
    // wave simply scans more of them (a chunk is the up to 64 keys of one cell
    // at rows row0 .. row0 + nk; the chunk -> (cell, row) map is uniform per
    // wave).  A chunk is read as the 64 keys from base = min(row0, nrows - 64),
    // so the loads of a chunk are four fixed offsets from one address and
    // never leave the store.
    int ccell = 0;
    int32_t c0 = 0;
    while (c0 < np - 1 && s_cpre[c0 + 1] == 0) c0++;
    const int64_t safe_row0 = nchunks > 0 ? s_r0[c0] : 0;
    auto fetch = [&](auto small, Chunk &ch) {
        constexpr bool SMALL = decltype(small)::value;
        int32_t gl = 0;
        if (lane == 0) gl = atomicAdd(&s_next, 1);
        const int32_t g = __builtin_amdgcn_readfirstlane(gl);
        ch.g = g;
        while (ccell < np - 1 && g >= s_cpre[ccell + 1]) ccell++;
        const bool live = g < nchunks;
        const int32_t key0 = (g - s_cpre[ccell]) * 64;
        const int32_t nk = live ? min(64, s_len[ccell] - key0) : 0;
        const int64_t row0 = live ? s_r0[ccell] + key0 : safe_row0;
        const int64_t base = SMALL ? 0 : (row0 < nrows - 64 ? row0 : nrows - 64);
        ch.base = base;
        ch.lo = (int32_t)(row0 - base);
        ch.hi = ch.lo + nk;
        load_chunk<SMALL>(codes, scales, base, nrows, row, col, lane, ch);
    };

    // Each wave keeps its own candidate list (no workgroup barrier in the scan,
    // so the waves drift apart and hide each other's memory latency).  Any
    // key above a threshold t with at least 128 scored keys at or below it can
    // be dropped.  Two such thresholds are kept: the wave's own 128th smallest
    // key, and the largest of the waves' published E8-th smallest keys (SW
    // waves x E8 keys at or below it).  Their minimum over the workgroup lives
    // in s_tau, which only decreases.
    // Each wave's list: wl[0, KMAX) holds its kept keys sorted ascending
    // (na of them, then NONE or larger keys already dropped), wl[KMAX, CAPW)
    // takes new keys (nb of them, at most 128).  Once more than 64 are
    // waiting they are merged into the kept ones (merge_new_keys).
    uint64_t *wl = cand + wave * CAPW;
    int na = 0, nb = 0;
    uint64_t tau_w = NONE;
    wl[lane] = NONE;
    wl[64 + lane] = NONE;
    // Folds this wave's thresholds into s_tau and drops the kept keys above
    // the result.
    auto refresh = [&]() {
        const uint64_t m = wave_max_u64(lane < SW ? s_e8[lane] : 0ull);
        const uint64_t t = tau_w < m ? tau_w : m;
        if (lane == 0) atomicMin(reinterpret_cast<unsigned long long *>(&s_tau), (unsigned long long)t);
        const uint64_t ts = __hip_atomic_load(&s_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const uint64_t cut = t < ts ? t : ts;
        int c = 0;
        for (int i = 0; i < na; i += 64) c += __popcll(__ballot(i + lane < na && wl[i + lane] <= cut));
        na = c;
    };
    auto wave_compact = [&]() {
        if (nb > 0) {
            const Kept k = merge_new_keys<E8>((lds_u64 *)wl, na, nb, (lds_u64 *)(s_e8 + wave), lane);
            na = k.na;
            nb = 0;
            tau_w = k.tau;
        }
        refresh();
    };
    auto score = [&](const Chunk &ch, bool merge = true) {
        int32_t dq[4], n12;
        score_chunk(ch, aq, dq, n12);
        const int32_t duq = dq[0];
        const float sc = ch.sc;
        const int32_t dot = 2 * duq - 3 * sq;
        const int32_t c2 = c2_base - 8 * n12;
        const float t1 = (sc * sc) * 0.25f * (float)c2;
        const float t3 = (sc * qs) * (float)dot;
        const float dist = t1 - t3 + 0.0f;
        const uint64_t k64 = ((uint64_t)fkey(dist) << 32) | (uint64_t)(uint32_t)(ch.base + lane);
        const uint64_t ts = __hip_atomic_load(&s_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const uint64_t tau = tau_w < ts ? tau_w : ts;
        const bool take = lane >= ch.lo && lane < ch.hi && k64 < tau;
        const uint64_t mask = __ballot(take);
        if (take) {
            const int pos = nb + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
            wl[KMAX + pos] = k64;
        }
        nb += __popcll(mask);
        if (merge && nb > 64) wave_compact();  // at most 128 new keys
    };

    // NF chunks per wave in flight: while one is scored the next NF - 1 load.
    // (Every step runs unconditionally: a chunk past the end has lo == hi and
    // scores nothing, and the loop body stays free of branches around loads.)
    // The empty asm with a memory clobber pins each fetch's loads above the
    // scoring that follows (the compiler would otherwise sink them to their
    // first use); nothing reads the loaded registers there, so no wait is added.
    auto scan = [&](auto small) {
        Chunk x[NF];
        // Phase A: each wave's first two chunks (1024 keys over the
        // workgroup), every key kept; each wave sorts its 128 and publishes
        // its E8-th smallest, and after one barrier every wave starts from the
        // largest of those.
#pragma unroll
        for (int i = 0; i < NF; i++) fetch(small, x[i]);
        asm volatile("" ::: "memory");
        score(x[0], false);
        score(x[1], false);
        wave_compact();
        fetch(small, x[0]);
        fetch(small, x[1]);
        asm volatile("" ::: "memory");
        __syncthreads();
        refresh();
        // Phase B: the rest, NF chunks per trip (x[2], ..., x[NF - 1], x[0],
        // x[1] hold this wave's next chunks in increasing order: once x[2]'s
        // is past the end, so are the others).
        while (x[2].g < nchunks) {
#pragma unroll
            for (int i = 0; i < NF; i++) {
                score(x[(i + 2) % NF]);
                fetch(small, x[(i + 2) % NF]);
                asm volatile("" ::: "memory");
            }
        }
    };
    if (nchunks > 0) {  // uniform over the workgroup
        if (nrows < 64)
            scan(std::integral_constant<bool, true>());
        else
            scan(std::integral_constant<bool, false>());
    }
    // Final: every wave sorts its list and keeps at most its best 128; the keys
    // at or below the final threshold (a superset of the query's top 128, at
    // most SW x 128) are gathered, and each one's rank among them (keys are
    // distinct: the index is part of the key) is its output position.
    wave_compact();
    __syncthreads();
    {
        const uint64_t m = wave_max_u64(lane < SW ? s_e8[lane] : 0ull);
        const uint64_t ts = s_tau;
        const uint64_t tfin = m < ts ? m : ts;
        for (int i = lane; i < na; i += 64) {
            const uint64_t e = wl[i];
            if (e <= tfin) fin[atomicAdd(&count, 1)] = e;
        }
    }
    __syncthreads();
    const int cnt = count;
    const float qn = s_qn;
    for (int t = tid; t < cnt; t += STH) {
        const uint64_t e = fin[t];
        int r = 0;
        for (int j = 0; j < cnt; j++) r += fin[j] < e;
        if (r < k) {
            const float v = qn + unfkey((uint32_t)(e >> 32));
            out_idx[q * k + r] = (int64_t)(uint32_t)e;
            out_dist[q * k + r] = v > 0.f ? v : 0.f;
        }
    }
    for (int j = cnt + tid; j < k; j += STH) {
        out_idx[q * k + j] = -1;
        out_dist[q * k + j] = __builtin_inff();
    }
}

// ---------------------------------------------------------------- cell-major search
//
// For batches whose queries probe the same cells several times over (the
// reference batches 2048-16384 queries per call and groups them by cell,
// ivf.rs:491-499, 528-686), each probed cell is read once for up to QG
// queries that probe it: one FP8 x FP4 MFMA already scores four query slots
// (build_aq / score_chunk), so the other three come free.
//   k_group_*       group the (query, probe) pairs by cell into units of at
//                   most QG queries of one cell;
//   k_search_cells  (persistent workgroups taking units from a counter) scans
//                   a unit's cell once, keeps each slot's exact top-KMAX of the
//                   cell as k_search keeps a query's, and writes it sorted to
//                   the pair's list parts[q nprobe + probe];
//   k_merge_parts   (one wave per query) merges the query's lists, keeping the
//                   KMAX smallest (bitonic split + merge per list), and writes
//                   k_search's outputs.
// The top-KMAX of the union of a query's cells lies in the union of the
// cells' top-KMAX, and every key is scored as k_search scores it, so the
// results are k_search's bit for bit.  Which queries share a unit depends on
// the order of atomics; the results do not.

constexpr int QG = 4;  // query slots per unit

struct CellUnit {
    int32_t cell, n;   // the cell and its query slots in use (1 .. QG)
    int32_t qp[QG];    // query * nprobe + probe slot of each
};

// A probe slot the scan covers: a cell id in [0, ncells), not repeated by an
// earlier slot of the same query (k_search scans such a cell once as well).
__device__ __forceinline__ bool probe_used(const int32_t *__restrict__ probes, int64_t q, int j, int32_t nprobe,
                                           int64_t ncells, int32_t &c) {
    c = probes[q * nprobe + j];
    if (c < 0 || c >= ncells) return false;
    for (int i = 0; i < j; i++)
        if (probes[q * nprobe + i] == c) return false;
    return true;
}

// Grouping of the (query, probe) pairs by cell, in four launches: cnt, fill
// (ncells ints each) and the per-query bounds qtau (nq) cleared; the used
// pairs counted per cell; the units per cell (ceil(cnt / QG)) scanned into
// ubase, with hdr[0] = units in all and hdr[1] = the scan's unit counter
// (0); the pairs scattered into their cells' units.
__global__ __launch_bounds__(256) void k_group_clear(int64_t ncells, int32_t nq, int32_t *cnt, int32_t *fill,
                                                     uint64_t *qtau) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < ncells) {
        cnt[i] = 0;
        fill[i] = 0;
    }
    if (i < nq) qtau[i] = NONE;
}

__global__ __launch_bounds__(256) void k_group_count(const int32_t *__restrict__ probes, int32_t nq, int32_t nprobe,
                                                     int64_t ncells, int32_t *cnt) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int32_t c;
    if (i < (int64_t)nq * nprobe && probe_used(probes, i / nprobe, (int)(i % nprobe), nprobe, ncells, c))
        atomicAdd(&cnt[c], 1);
}

// grid: 1 workgroup of GT threads, each a contiguous range of cells; the
// ranges' sums are scanned in LDS.
constexpr int GT = 1024;
__global__ __launch_bounds__(GT) void k_group_scan(const int32_t *__restrict__ cnt, int64_t ncells,
                                                   int32_t *__restrict__ ubase, int32_t *hdr) {
    __shared__ int32_t s[GT];
    const int tid = threadIdx.x;
    const int64_t per = (ncells + GT - 1) / GT;
    const int64_t c0 = min(ncells, (int64_t)tid * per), c1 = min(ncells, c0 + per);
    int32_t local = 0;
    for (int64_t c = c0; c < c1; c++) local += (cnt[c] + QG - 1) / QG;
    s[tid] = local;
    __syncthreads();
    for (int o = 1; o < GT; o <<= 1) {
        const int32_t v = tid >= o ? s[tid - o] : 0;
        __syncthreads();
        s[tid] += v;
        __syncthreads();
    }
    int32_t run = s[tid] - local;
    for (int64_t c = c0; c < c1; c++) {
        ubase[c] = run;
        run += (cnt[c] + QG - 1) / QG;
    }
    if (tid == GT - 1) {
        hdr[0] = s[GT - 1];
        hdr[1] = 0;
    }
}

__global__ __launch_bounds__(256) void k_group_scatter(const int32_t *__restrict__ probes, int32_t nq, int32_t nprobe,
                                                       int64_t ncells, const int32_t *__restrict__ cnt,
                                                       int32_t *fill, const int32_t *__restrict__ ubase,
                                                       CellUnit *units) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int32_t c;
    if (i >= (int64_t)nq * nprobe || !probe_used(probes, i / nprobe, (int)(i % nprobe), nprobe, ncells, c)) return;
    const int32_t pos = atomicAdd(&fill[c], 1);
    CellUnit &u = units[ubase[c] + pos / QG];
    u.qp[pos % QG] = (int32_t)i;
    if (pos % QG == 0) {
        u.cell = c;
        u.n = min(QG, cnt[c] - pos);
    }
}

// Merges the sorted KMAX-list at B into the sorted one at A, keeping the KMAX
// smallest (sorted) at A: the minimum of each of A's keys and B's mirrored key
// is a bitonic sequence holding the KMAX smallest of both, which a bitonic
// merge sorts.
__device__ __forceinline__ void merge_lists(lds_u64 *A, const lds_u64 *B, int lane) {
    uint64_t c[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const uint64_t a = A[r * 64 + lane];
        const uint64_t b = shfl_xor_u64(B[(1 - r) * 64 + lane], 63, lane);  // B's key 127 - (64 r + lane)
        c[r] = a < b ? a : b;
    }
    bitonic_stage<2, 128, 64>(c, lane);
    A[lane] = c[0];
    A[64 + lane] = c[1];
}

// grid: persistent workgroups of CTH threads taking units from hdr[1] until
// hdr[0] are done.  parts [nq nprobe][KMAX] keys (ordered dist bits << 32 |
// row), each pair's list sorted ascending, NONE-padded.  qtau [nq]: a bound on
// each query's k-th smallest key over all its cells (keys are distinct, so
// the k-th smallest key of any one of its cells bounds it); every finished
// (query, cell) list lowers it, and every later unit of the query drops keys
// at or above it from the start.  A bound read stale is larger, never wrong.
// Two waves per workgroup, six workgroups per CU (12 waves; the register
// budget is capped at 168 VGPRs for that and 32 spill): one workgroup's unit
// set-up and final merges then idle a sixth of the CU's loads in flight, and
// each unit streams twice as long as with four waves.  4,096 queries x 8
// probes: 1.62 ms, against 1.74 ms with four-wave workgroups three per CU,
// 1.88 ms two per CU at 207 VGPRs, 1.98 ms four per CU (72 spilled) and
// 1.67 ms with one-wave workgroups twelve per CU.
constexpr int CW = 2;                       // waves per cell-major workgroup
constexpr int CTH = CW * 64;
constexpr int E8C = (KMAX + CW - 1) / CW;   // each wave's published rank
__global__ __launch_bounds__(CTH) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_search_cells(const uint8_t *codes, const float *scales,
                                                      const int64_t *__restrict__ cell_start, int64_t ncells,
                                                      const float *__restrict__ queries, int32_t nprobe, int32_t k,
                                                      const CellUnit *__restrict__ units, int32_t *hdr,
                                                      uint64_t *qtau, uint64_t *__restrict__ parts) {
    __shared__ uint64_t cand[QG][CW * CAPW];  // per slot, per-wave candidate lists
    __shared__ uint64_t s_tau[QG];            // per slot shared threshold (only decreases within a unit)
    __shared__ uint64_t s_e8[QG][CW];
    __shared__ int16_t s_Q[QG * D];
    __shared__ float s_qs[QG];
    __shared__ int32_t s_sq[QG];
    __shared__ int32_t s_next, s_unit, s_len;
    __shared__ int64_t s_r0;
    __shared__ CellUnit s_u;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = lane >> 4, col = lane & 15;
    const int32_t n_units = hdr[0];
    const int64_t nrows = cell_start[ncells];
    const int32_t c2_base = 9 * D;

    for (;;) {
        if (tid == 0) s_unit = atomicAdd(&hdr[1], 1);
        __syncthreads();
        const int32_t u = s_unit;
        if (u >= n_units) break;  // uniform over the workgroup
        if (tid < (int)(sizeof(CellUnit) / 4))
            reinterpret_cast<int32_t *>(&s_u)[tid] = reinterpret_cast<const int32_t *>(units + u)[tid];
        __syncthreads();
        const int n = s_u.n;
        if (tid == 0) {
            const int64_t r0 = cell_start[s_u.cell];
            s_r0 = r0;
            s_len = (int32_t)(cell_start[s_u.cell + 1] - r0);
            s_next = 0;
        }
        // An absent slot takes nothing (every key compares above 0).
        if (tid < QG)
            s_tau[tid] = tid < n ? __hip_atomic_load(&qtau[s_u.qp[tid] / nprobe], __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)
                                 : 0ull;
        if (tid < QG * CW) s_e8[tid / CW][tid % CW] = NONE;
        for (int s = wave; s < n; s += CW) {
            const QInfo qi = quantize_query(queries + (int64_t)(s_u.qp[s] / nprobe) * D, lane, s_Q + s * D);
            if (lane == 0) {
                s_qs[s] = qi.qs;
                s_sq[s] = qi.sq;
            }
        }
        __syncthreads();

        v8i aq[2];
        build_aq(s_Q, n, row, col, aq);
        float qs[QG];
        int32_t sq[QG];
#pragma unroll
        for (int s = 0; s < QG; s++) {
            qs[s] = s_qs[s < n ? s : 0];
            sq[s] = s_sq[s < n ? s : 0];
        }
        const int64_t r0 = s_r0;
        const int32_t len = s_len;
        const int32_t nchunks = (len + 63) / 64;

        // A store of fewer than 64 rows takes the clamped loads (SMALL).
        auto fetch = [&](auto small, Chunk &ch) {
            constexpr bool SMALL = decltype(small)::value;
            int32_t gl = 0;
            if (lane == 0) gl = atomicAdd(&s_next, 1);
            const int32_t g = __builtin_amdgcn_readfirstlane(gl);
            ch.g = g;
            const bool live = g < nchunks;
            const int32_t key0 = g * 64;
            const int32_t nk = live ? min(64, len - key0) : 0;
            const int64_t row0 = live ? r0 + key0 : r0;
            const int64_t base = SMALL ? 0 : (row0 < nrows - 64 ? row0 : nrows - 64);
            ch.base = base;
            ch.lo = (int32_t)(row0 - base);
            ch.hi = ch.lo + nk;
            load_chunk<SMALL>(codes, scales, base, nrows, row, col, lane, ch);
        };

        int na[QG], nb[QG];
        uint64_t tau_w[QG];
#pragma unroll
        for (int s = 0; s < QG; s++) {
            na[s] = 0;
            nb[s] = 0;
            tau_w[s] = NONE;
            uint64_t *wl = cand[s] + wave * CAPW;
            wl[lane] = NONE;
            wl[64 + lane] = NONE;
        }
        auto refresh = [&](int s) {
            const uint64_t m = wave_max_u64(lane < CW ? s_e8[s][lane] : 0ull);
            const uint64_t t = tau_w[s] < m ? tau_w[s] : m;
            if (lane == 0) atomicMin(reinterpret_cast<unsigned long long *>(&s_tau[s]), (unsigned long long)t);
            const uint64_t ts = __hip_atomic_load(&s_tau[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            const uint64_t cut = t < ts ? t : ts;
            const uint64_t *wl = cand[s] + wave * CAPW;
            int c = 0;
            for (int i = 0; i < na[s]; i += 64) c += __popcll(__ballot(i + lane < na[s] && wl[i + lane] <= cut));
            na[s] = c;
        };
        auto compact = [&](int s) {
            if (nb[s] > 0) {
                const Kept kk = merge_new_keys<E8C>((lds_u64 *)(cand[s] + wave * CAPW), na[s], nb[s],
                                                    (lds_u64 *)(&s_e8[s][wave]), lane);
                na[s] = kk.na;
                nb[s] = 0;
                tau_w[s] = kk.tau;
            }
            refresh(s);
        };
        auto score = [&](const Chunk &ch, bool merge) {
            int32_t dq[4], n12;
            score_chunk(ch, aq, dq, n12);
            const float sc = ch.sc;
            const int32_t c2 = c2_base - 8 * n12;
            const float t1 = (sc * sc) * 0.25f * (float)c2;
            const uint32_t kidx = (uint32_t)(ch.base + lane);
            const bool in = lane >= ch.lo && lane < ch.hi;
#pragma unroll
            for (int s = 0; s < QG; s++) {
                if (s >= n) break;  // uniform
                const int32_t dot = 2 * dq[s] - 3 * sq[s];
                const float t3 = (sc * qs[s]) * (float)dot;
                const float dist = t1 - t3 + 0.0f;
                const uint64_t k64 = ((uint64_t)fkey(dist) << 32) | (uint64_t)kidx;
                const uint64_t ts = __hip_atomic_load(&s_tau[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                const uint64_t tau = tau_w[s] < ts ? tau_w[s] : ts;
                const bool take = in && k64 < tau;
                const uint64_t mask = __ballot(take);
                if (take) {
                    const int pos = nb[s] + (int)__builtin_amdgcn_mbcnt_hi(
                                                (uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
                    cand[s][wave * CAPW + KMAX + pos] = k64;
                }
                nb[s] += __popcll(mask);
                if (merge && nb[s] > 64) compact(s);  // at most 128 new keys
            }
        };

        // As k_search's scan: each wave's first two chunks kept (below the
        // query's bound), a compaction and one barrier, then NF chunks in
        // flight per trip.
        auto scan = [&](auto small) {
            Chunk x[NF];
#pragma unroll
            for (int i = 0; i < NF; i++) fetch(small, x[i]);
            asm volatile("" ::: "memory");
            score(x[0], false);
            score(x[1], false);
#pragma unroll
            for (int s = 0; s < QG; s++)
                if (s < n) compact(s);
            fetch(small, x[0]);
            fetch(small, x[1]);
            asm volatile("" ::: "memory");
            __syncthreads();
#pragma unroll
            for (int s = 0; s < QG; s++)
                if (s < n) refresh(s);
            while (x[2].g < nchunks) {
#pragma unroll
                for (int i = 0; i < NF; i++) {
                    score(x[(i + 2) % NF], true);
                    fetch(small, x[(i + 2) % NF]);
                    asm volatile("" ::: "memory");
                }
            }
        };
        if (nchunks > 0) {  // uniform
            if (nrows < 64)
                scan(std::integral_constant<bool, true>());
            else
                scan(std::integral_constant<bool, false>());
        }
        // Each wave's kept list of each slot, sorted and NONE-padded to KMAX;
        // then per slot a merge tree over the waves (wave w takes w + 1, then
        // w + 2), and the slot's list goes to its pair's part; its k-th key
        // lowers the query's bound.
#pragma unroll
        for (int s = 0; s < QG; s++) {
            if (s >= n) break;
            compact(s);
            uint64_t *wl = cand[s] + wave * CAPW;
            const uint64_t a0 = lane < na[s] ? wl[lane] : NONE, a1 = 64 + lane < na[s] ? wl[64 + lane] : NONE;
            wl[lane] = a0;
            wl[64 + lane] = a1;
        }
        __syncthreads();
#pragma unroll
        for (int step = 1; step < CW; step <<= 1) {
            if ((wave & (2 * step - 1)) == 0)
                for (int s = 0; s < n; s++)
                    merge_lists((lds_u64 *)(cand[s] + wave * CAPW), (const lds_u64 *)(cand[s] + (wave + step) * CAPW),
                                lane);
            __syncthreads();
        }
        for (int i = tid; i < n * KMAX; i += CTH) {
            const int s = i / KMAX, e = i % KMAX;
            parts[(int64_t)s_u.qp[s] * KMAX + e] = cand[s][e];
        }
        if (tid < n) {
            const uint64_t kth = cand[tid][k - 1];
            if (kth != NONE)
                __hip_atomic_fetch_min(&qtau[s_u.qp[tid] / nprobe], kth, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();  // LDS is reused by the next unit
    }
}

// grid: one 64-thread workgroup per query.  Merges the query's per-probe
// lists (the slots the grouping used; others are skipped) and writes
// k_search's outputs: ranks 0 .. k - 1, max(|Q qs|^2 + dist, 0), -1 / +inf
// padding.
__global__ __launch_bounds__(64) void k_merge_parts(const uint64_t *__restrict__ parts,
                                                    const int32_t *__restrict__ probes, int32_t nprobe,
                                                    int64_t ncells, const float *__restrict__ queries, int32_t k,
                                                    int64_t *__restrict__ out_idx, float *__restrict__ out_dist) {
    __shared__ int16_t sQ[D];
    __shared__ uint64_t acc[KMAX], lst[KMAX];
    const int lane = threadIdx.x;
    const int64_t q = blockIdx.x;
    const QInfo qi = quantize_query(queries + q * D, lane, sQ);
    acc[lane] = NONE;
    acc[64 + lane] = NONE;
    for (int j = 0; j < nprobe; j++) {
        int32_t c;
        if (!probe_used(probes, q, j, nprobe, ncells, c)) continue;  // uniform
        const uint64_t *L = parts + (q * nprobe + j) * KMAX;
        lst[lane] = L[lane];
        lst[64 + lane] = L[64 + lane];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        merge_lists((lds_u64 *)acc, (const lds_u64 *)lst, lane);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int rank = r * 64 + lane;
        if (rank >= k) continue;
        const uint64_t e = acc[rank];
        if (e != NONE) {
            const float v = qi.qn + unfkey((uint32_t)(e >> 32));
            out_idx[q * k + rank] = (int64_t)(uint32_t)e;
            out_dist[q * k + rank] = v > 0.f ? v : 0.f;
        } else {
            out_idx[q * k + rank] = -1;
            out_dist[q * k + rank] = __builtin_inff();
        }
    }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Scan order of st_knn_search_ivf_2bit (st_knn_set_scan_order): 0 chooses,
// 1 query-major (k_search), 2 cell-major.
int32_t g_scan_order = 0;

}  // namespace

extern "C" st_status st_knn_quantize_2bit(const float *keys, int64_t n, int64_t d, uint8_t *codes, float *scales,
                                          st_stream stream) {
    st::clear_error();
    if (!keys || !codes || !scales) return st::fail(ST_ERR_INVALID, "quantize: NULL buffer");
    if (n < 0 || d <= 0 || d % 16 != 0)
        return st::fail(ST_ERR_INVALID, "quantised keys need d %% 16 == 0 (got d = %lld)", (long long)d);
    if ((reinterpret_cast<uintptr_t>(codes) & 3) != 0) return st::fail(ST_ERR_INVALID, "codes must be 4-byte aligned");
    if (n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st::stream_of(stream), keys, n,
                       (int32_t)d, codes, scales);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_knn_key_norms_2bit(const uint8_t *codes, const float *scales, int64_t n, int64_t d,
                                           float *norms, st_stream stream) {
    st::clear_error();
    if (!codes || !scales || !norms) return st::fail(ST_ERR_INVALID, "key_norms: NULL buffer");
    if (n < 0 || d <= 0 || d % 16 != 0)
        return st::fail(ST_ERR_INVALID, "quantised keys need d %% 16 == 0 (got d = %lld)", (long long)d);
    if (n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    if (cdiv(n, 256) > INT32_MAX) return st::fail(ST_ERR_INVALID, "key_norms: too many rows for one call");
    hipLaunchKernelGGL(k_key_norms, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st::stream_of(stream), codes, scales,
                       n, (int32_t)d, norms);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_knn_synth_store_2bit(uint64_t seed, int64_t row0, int64_t n, int64_t d, uint8_t *codes,
                                             float *scales, st_stream stream) {
    st::clear_error();
    if (!codes || !scales) return st::fail(ST_ERR_INVALID, "synth: NULL buffer");
    if (n < 0 || row0 < 0 || d != D) return st::fail(ST_ERR_INVALID, "synth: needs n >= 0 and d == %d", D);
    if ((reinterpret_cast<uintptr_t>(codes) & 3) != 0) return st::fail(ST_ERR_INVALID, "codes must be 4-byte aligned");
    if (n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    if (cdiv(n, 256) > INT32_MAX) return st::fail(ST_ERR_INVALID, "synth: too many rows for one call");
    hipLaunchKernelGGL(k_synth_store, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st::stream_of(stream), seed, row0,
                       n, (int32_t)d, codes, scales);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

// Benchmark/test support: the f32 keys st_knn_synth_store_2bit quantises.
extern "C" st_status st_knn_synth_keys_f32(uint64_t seed, int64_t row0, int64_t n, int64_t d, float *keys,
                                           st_stream stream) {
    st::clear_error();
    if (!keys) return st::fail(ST_ERR_INVALID, "synth keys: NULL buffer");
    if (n < 0 || row0 < 0 || d != D) return st::fail(ST_ERR_INVALID, "synth keys: needs n >= 0 and d == %d", D);
    if (n == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    hipLaunchKernelGGL(k_synth_keys, dim3((unsigned)cdiv(n * d, 256)), dim3(256), 0, st::stream_of(stream), seed,
                       row0, n, (int32_t)d, keys);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_knn_search_ivf_2bit(const uint8_t *codes, const float *scales, const int64_t *cell_start,
                                            int64_t ncells, int64_t max_cell, const float *queries,
                                            const int32_t *probes, int64_t nq, int64_t nprobe, int64_t d,
                                            int64_t k, int64_t *out_idx, float *out_dist, st_stream stream) {
    st::clear_error();
    if (!codes || !scales || !cell_start || !queries || !probes || !out_idx || !out_dist)
        return st::fail(ST_ERR_INVALID, "search_ivf: NULL buffer");
    if (d != D) return st::fail(ST_ERR_INVALID, "search_ivf: the 2-bit scan is built for d == %d (got %lld)", D, (long long)d);
    if (nq < 0 || ncells < 1 || max_cell < 0) return st::fail(ST_ERR_INVALID, "search_ivf: bad nq, ncells or max_cell");
    if (nprobe < 1 || nprobe > ncells || nprobe > PROBE_MAX)
        return st::fail(ST_ERR_INVALID, "search_ivf: nprobe must be in 1..=min(ncells, %d) (got %lld)", PROBE_MAX,
                        (long long)nprobe);
    if (k < 1 || k > KMAX) return st::fail(ST_ERR_INVALID, "search_ivf: k must be in 1..=%d (got %lld)", KMAX, (long long)k);
    if ((reinterpret_cast<uintptr_t>(codes) & 15) != 0 || (reinterpret_cast<uintptr_t>(queries) & 15) != 0)
        return st::fail(ST_ERR_INVALID, "search_ivf: codes and queries must be 16-byte aligned");
    if (nq == 0) return ST_OK;
    if (nq > INT32_MAX / PROBE_MAX) return st::fail(ST_ERR_INVALID, "search_ivf: too many queries for one call");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const hipStream_t s = st::stream_of(stream);
    // Query-major (a workgroup per query, each probed cell read once per
    // query that probes it) unless the batch probes the cells 2/3 of a time
    // or more on average: then cell-major, each probed cell read once for up
    // to QG queries (12,288 cells x 8 probes: 0.42 against 0.48 ms at 512
    // queries, 0.82 against 0.78 ms at 1,024).
    const int64_t npairs = nq * nprobe;
    const bool cells = g_scan_order == 2 || (g_scan_order == 0 && 3 * npairs >= 2 * ncells);
    if (!cells) {
        hipLaunchKernelGGL(k_search<false>, dim3((unsigned)nq), dim3(STH), 0, s, codes, scales, cell_start, ncells,
                           queries, probes, (int32_t)nq, (int32_t)nprobe, (int32_t)k, out_idx, out_dist, nullptr,
                           (int64_t)0, (int64_t)0);
        ST_LAUNCH_CHECK();
        return ST_OK;
    }
    if (ncells > INT32_MAX) return st::fail(ST_ERR_INVALID, "search_ivf: too many cells for the cell-major scan");
    // Scratch: per-cell counts, fill counters and unit offsets, the unit
    // header, the units (at most one per pair) and one KMAX list per pair.
    const size_t cells_b = (size_t)(3 * ncells + 2) * sizeof(int32_t);
    const size_t qtau_off = (cells_b + 15) & ~(size_t)15;
    const size_t units_off = qtau_off + (size_t)nq * sizeof(uint64_t);
    const size_t parts_off = (units_off + (size_t)npairs * sizeof(CellUnit) + 255) & ~(size_t)255;
    const size_t bytes = parts_off + (size_t)npairs * KMAX * sizeof(uint64_t);
    char *base = static_cast<char *>(st::scratch(st::SCRATCH_KNN, bytes, s));
    if (!base) return st::scratch_status();
    int32_t *cnt = reinterpret_cast<int32_t *>(base), *fill = cnt + ncells, *ubase = fill + ncells,
            *hdr = ubase + ncells;
    uint64_t *qtau = reinterpret_cast<uint64_t *>(base + qtau_off);
    CellUnit *units = reinterpret_cast<CellUnit *>(base + units_off);
    uint64_t *parts = reinterpret_cast<uint64_t *>(base + parts_off);
    const unsigned pb = (unsigned)cdiv(npairs, 256);
    hipLaunchKernelGGL(k_group_clear, dim3((unsigned)cdiv(std::max<int64_t>(ncells, nq), 256)), dim3(256), 0, s,
                       ncells, (int32_t)nq, cnt, fill, qtau);
    hipLaunchKernelGGL(k_group_count, dim3(pb), dim3(256), 0, s, probes, (int32_t)nq, (int32_t)nprobe, ncells, cnt);
    hipLaunchKernelGGL(k_group_scan, dim3(1), dim3(GT), 0, s, cnt, ncells, ubase, hdr);
    hipLaunchKernelGGL(k_group_scatter, dim3(pb), dim3(256), 0, s, probes, (int32_t)nq, (int32_t)nprobe, ncells, cnt,
                       fill, ubase, units);
    ST_LAUNCH_CHECK();
    const int cus = st::device_cus();
    // Persistent workgroups, six per CU (those that find no unit left exit).
    const unsigned wgs = (unsigned)std::min<int64_t>(npairs, 6 * (int64_t)cus);
    hipLaunchKernelGGL(k_search_cells, dim3(wgs), dim3(CTH), 0, s, codes, scales, cell_start, ncells, queries,
                       (int32_t)nprobe, (int32_t)k, units, hdr, qtau, parts);
    ST_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_merge_parts, dim3((unsigned)nq), dim3(64), 0, s, parts, probes, (int32_t)nprobe, ncells,
                       queries, (int32_t)k, out_idx, out_dist);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_knn_set_scan_order(int32_t order) {
    st::clear_error();
    if (order < 0 || order > 2) return st::fail(ST_ERR_INVALID, "scan order must be 0, 1 or 2 (got %d)", order);
    g_scan_order = order;
    return ST_OK;
}

extern "C" st_status st_knn_search_masked_2bit(const uint8_t *codes, const float *scales, int64_t nkeys,
                                               const float *queries, const int64_t *lohi, int64_t always,
                                               int64_t nq, int64_t d, int64_t k, int64_t *out_idx, float *out_dist,
                                               st_stream stream) {
    st::clear_error();
    if (!codes || !scales || !queries || !lohi || !out_idx || !out_dist)
        return st::fail(ST_ERR_INVALID, "search_masked: NULL buffer");
    if (d != D) return st::fail(ST_ERR_INVALID, "search_masked: the 2-bit scan is built for d == %d (got %lld)", D,
                                (long long)d);
    if (nkeys < KMAX) return st::fail(ST_ERR_INVALID, "need at least %d keys", KMAX);  // knn.rs:305
    if (nkeys >= (1ll << 31)) return st::fail(ST_ERR_INVALID, "search_masked: the store must hold fewer than 2^31 keys");
    if (nq < 0 || always < 0) return st::fail(ST_ERR_INVALID, "search_masked: bad nq or always");
    if (k < 1 || k > KMAX) return st::fail(ST_ERR_INVALID, "search_masked: k must be in 1..=%d (got %lld)", KMAX,
                                           (long long)k);
    if ((reinterpret_cast<uintptr_t>(codes) & 15) != 0 || (reinterpret_cast<uintptr_t>(queries) & 15) != 0)
        return st::fail(ST_ERR_INVALID, "search_masked: codes and queries must be 16-byte aligned");
    if (nq == 0) return ST_OK;
    if (nq > INT32_MAX) return st::fail(ST_ERR_INVALID, "search_masked: too many queries for one call");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    hipLaunchKernelGGL(k_search<true>, dim3((unsigned)nq), dim3(STH), 0, st::stream_of(stream), codes, scales,
                       nullptr, (int64_t)0, queries, nullptr, (int32_t)nq, 0, (int32_t)k, out_idx, out_dist, lohi,
                       always, nkeys);
    ST_LAUNCH_CHECK();
    return ST_OK;
}
