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
// Search design: one 1024-thread workgroup (16 wave64s) per query streams the
// concatenation of its probed cells, 1024 keys (64 KB of codes) per iteration
// with the next iteration's loads in flight.  Lane l handles bytes 16*(l%4)..
// of a key (4 of its 16 code dwords), so a wave's loads are fully coalesced
// 1 KB rows and each lane keeps only its quarter of the query in registers.
// The query is held as balanced base-16 digits (Q = d0 + 16 d1 + 256 d2 +
// 4096 d3, d in [-8, 7]); per code dword two masks give the codes as 4-bit
// nibbles and eight v_dot8_i32_i4 (one per digit and nibble set) accumulate
// the exact dot, one popcount gives c2.  The four quarter sums are combined
// with two butterfly shuffles (integers: exact in any order).
//
// Top-k: each wave appends candidates with key64 = (ordered dist bits << 32 |
// index) below its threshold to its own LDS list (ballot + mbcnt, no atomics,
// no workgroup barrier in the scan); when the list fills (or after the first
// 256 candidates) a wave-level bitonic sort keeps its 128 smallest and its
// threshold becomes the 128th, published to the workgroup through an LDS
// atomicMin.  Only keys with at least 128 smaller keys already seen are
// dropped, so the exact top-128 survives whatever the order, and the final
// sort makes the result deterministic.  Cells that other queries of the
// batch also probe are scanned first, so their bytes are read while the other
// workgroups still find them in the MALL.
#include <cstring>

#include "common.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 256;          // key width handled by the scan
constexpr int DW = D / 16;      // code dwords per key
constexpr int KMAX = 128;       // neighbours kept per query (knn.rs:21)
constexpr int CAPW = 512;       // LDS candidate list per wave (entries)
constexpr int FIN = 4096;       // LDS starting set + final gather (entries)
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

constexpr int SW = 16;          // waves per search workgroup
constexpr int STH = SW * 64;    // threads per search workgroup (one workgroup per query)
constexpr int KPI = STH;        // keys scanned per iteration: 4 lanes per key, 4 sub-steps

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sorts buf[0..n) ascending (n a power of two) with all threads of the block.
__device__ void bitonic_sort(uint64_t *buf, int n) {
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < n; i += nt) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = buf[i], b = buf[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        buf[i] = b;
                        buf[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Sorts buf[0..n) ascending (n a power of two) within one wave: LDS operations
// of a wave complete in order, so the stages need no barrier, only a fence that
// keeps the compiler from reordering them.
__device__ void wave_sort(uint64_t *buf, int n, int lane) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = lane; i < n; i += 64) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = buf[i], b = buf[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        buf[i] = b;
                        buf[ixj] = a;
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
    }
}

__device__ __forceinline__ int pow2_at_least(int x) {
    int n = KMAX;
    while (n < x) n <<= 1;
    return n;
}

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Sum over the four 16-lane rows of a wave (every lane gets its column's sum),
// with the gfx950 row swaps: x + swap16(x), then + swap32.
__device__ __forceinline__ int32_t rows_sum(int32_t x) {
    auto a = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    x = (int32_t)(a[0] + a[1]);
    auto b = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return (int32_t)(b[0] + b[1]);
}

// grid: one workgroup of 1024 threads per query.
__global__ __launch_bounds__(STH) void k_search(const uint8_t *codes, const float *scales,
                                                const int64_t *__restrict__ cell_start, int64_t ncells,
                                                const float *__restrict__ queries, const int32_t *__restrict__ probes,
                                                int32_t nq, int32_t nprobe, int32_t k, int64_t *__restrict__ out_idx,
                                                float *__restrict__ out_dist) {
    __shared__ uint64_t cand[SW * CAPW];  // per-wave candidate lists
    __shared__ uint64_t fin[FIN];         // the starting set and the final gather
    __shared__ uint64_t s_tau;            // min over the waves' thresholds
    __shared__ int16_t s_Q[D];
    __shared__ float s_qs, s_qn;
    __shared__ int32_t s_sq, s_np, count;
    __shared__ int32_t s_cell[PROBE_MAX], s_share[PROBE_MAX];
    __shared__ int64_t s_r0[PROBE_MAX];
    __shared__ int32_t s_len[PROBE_MAX], s_cpre[PROBE_MAX + 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t q = blockIdx.x;

    if (wave == 0) {
        // Query quantisation: qs = 2^(E-14) with max|q| = m 2^E, Q = clamp(rint(q / qs), -16384, 16383).
        const float4 v = reinterpret_cast<const float4 *>(queries + q * D)[lane];
        const float x[4] = {v.x, v.y, v.z, v.w};
        const float mx = wave_max(fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))));
        float qs = 1.f, inv = 1.f;
        if (mx > 0.f) {
            int e;
            frexpf(mx, &e);
            qs = ldexpf(1.f, e - 14);
            inv = ldexpf(1.f, 14 - e);
        }
        int32_t sq = 0;
        double sq2 = 0.0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int32_t Q = (int32_t)fminf(fmaxf(rintf(x[t] * inv), -16384.f), 16383.f);
            sq += Q;
            sq2 += (double)Q * (double)Q;
            s_Q[4 * lane + t] = (int16_t)Q;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            sq += __shfl_xor(sq, o, 64);
            sq2 += __shfl_xor(sq2, o, 64);
        }
        if (lane == 0) {
            s_qs = qs;
            s_qn = (float)sq2 * (qs * qs);
            s_sq = sq;
        }
    } else {
        // How many (query, probe) pairs of the whole batch scan each probed cell.
        for (int j = wave - 1; j < nprobe; j += SW - 1) {
            const int32_t cell = probes[q * nprobe + j];
            int cnt = 0;
            for (int64_t i = lane; i < (int64_t)nq * nprobe; i += 64) cnt += probes[i] == cell;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
            if (lane == 0) {
                s_cell[j] = cell;
                s_share[j] = cnt;
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        // Cells scanned by several queries of the batch first (their bytes are
        // then read while still in the MALL), a repeated cell once, invalid ids
        // skipped; s_cpre counts 64-key chunks.
        int order[PROBE_MAX];
        for (int j = 0; j < nprobe; j++) {
            int i = j;
            while (i > 0 && (s_share[order[i - 1]] < s_share[j] ||
                             (s_share[order[i - 1]] == s_share[j] && s_cell[order[i - 1]] > s_cell[j]))) {
                order[i] = order[i - 1];
                i--;
            }
            order[i] = j;
        }
        int np = 0;
        int32_t prev = -1;
        s_cpre[0] = 0;
        for (int i = 0; i < nprobe; i++) {
            const int32_t c = s_cell[order[i]];
            if (c < 0 || c >= ncells || c == prev) continue;
            prev = c;
            const int64_t len = cell_start[c + 1] - cell_start[c];
            s_r0[np] = cell_start[c];
            s_len[np] = (int32_t)len;
            s_cpre[np + 1] = s_cpre[np] + (int32_t)((len + 63) / 64);
            np++;
        }
        s_np = np;
        count = 0;
        s_tau = NONE;
    }
    __syncthreads();

    // Matrix-core operands.  The key side (B, 128 x 16 per k-step, FP4 e2m1):
    // a code u kept in the low two bits of a nibble is the e2m1 number u / 2
    // (0, 0.5, 1, 1.5), so w & 0x33333333 and (w >> 2) & 0x33333333 are ready
    // operands: nibble j of the first is code 2j of code dword w, of the
    // second code 2j + 1.  Lane l supplies column l % 16 (a key) and the 32
    // values of k-block l / 16; at k-step m (0, 1) they are dims
    // 16 (4 (l/16) + 2m) + [0, 2, .., 14], then + 1, then the same for code
    // dword 4 (l/16) + 2m + 1: FP4 nibble n of k-block h is k = 32 h + n.  The
    // query side (A, FP8 e4m3) orders k differently: byte n of lane group g is
    // k = 16 g + n for n < 16 and k = 64 + 16 g + (n - 16) above.  Row p < 4
    // holds balanced base-16 digit p of Q (Q = d0 + 16 d1 + 256 d2 + 4096 d3,
    // d in [-8, 7], exact in FP8) at the dim its k pairs with; rows 4..15 are
    // zero.  Products and sums are small half-integers, exact in the f32
    // accumulator.
    const int row = lane >> 4, col = lane & 15;
    v8i aq[2];
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
                int32_t Q = s_Q[16 * dword + code];
                int32_t dgt = 0;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int32_t d = p < 3 ? ((Q + 8) & 15) - 8 : Q;
                    if (p == col) dgt = d;
                    Q = (Q - d) >> 4;
                }
                f[e] = col < 4 ? (float)dgt : 0.f;
            }
            int32_t word = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
            word = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], word, true);
            aq[m][v] = word;
        }
    }
    const float qs = s_qs;
    const int32_t sq = s_sq;
    const int np = s_np;
    const int32_t nchunks = s_cpre[np];
    const int32_t c2_base = 9 * D;

    // Wave w scans chunks w, w + 16, ... of the query's cells taken in order (a
    // chunk is 64 consecutive keys of one cell; the chunk -> (cell, row) map is
    // uniform per wave).  For group G (keys 16G..16G+15 of the chunk) lane l
    // loads bytes 16 (l/16) .. of key 16G + l%16: the 16-byte key operand of
    // matrix-core column l%16, k-block l/16, for the four k-steps; a wave's
    // load reads 1 KB of consecutive codes.  Past a cell's end (or the last
    // chunk) lanes read the chunk's first key and are ignored.
    int ccell = 0;
    struct Chunk {
        uint4 c[4];
        float sc;
        int64_t row0;
        int32_t nk;
    };
    int32_t c0 = 0;
    while (c0 < np - 1 && s_cpre[c0 + 1] == 0) c0++;
    const int64_t safe_row0 = nchunks > 0 ? s_r0[c0] : 0;
    auto fetch = [&](int32_t g, Chunk &ch) {
        while (ccell < np - 1 && g >= s_cpre[ccell + 1]) ccell++;
        const bool live = g < nchunks;
        const int32_t key0 = (g - s_cpre[ccell]) * 64;
        const int32_t nk = live ? min(64, s_len[ccell] - key0) : 0;
        ch.row0 = live ? s_r0[ccell] + key0 : safe_row0;
        ch.nk = nk;
        const uint4 *cb = reinterpret_cast<const uint4 *>(codes + ch.row0 * (D / 4));
#pragma unroll
        for (int G = 0; G < 4; G++) {
            const int32_t kk = 16 * G + col;
            ch.c[G] = cb[(kk < nk ? kk : 0) * 4 + row];
        }
        ch.sc = scales[ch.row0 + (lane < nk ? lane : 0)];  // lane l scores chunk key l
    };

    // Each wave keeps its own candidate list (no workgroup barrier in the scan,
    // so the 16 waves drift apart and hide each other's memory latency).  A
    // wave's threshold is the 128th smallest key it has kept; the smallest of
    // all waves' thresholds (shared through LDS) is also valid: the wave that
    // owns it holds 128 keys at or below it.
    uint64_t *wl = cand + wave * CAPW;
    int wcount = 0;
    uint64_t tau_w = NONE;
    auto wave_compact = [&]() {
        const int n = pow2_at_least(wcount);
        for (int i = wcount + lane; i < n; i += 64) wl[i] = NONE;
        wave_sort(wl, n, lane);
        if (wcount >= KMAX) {
            tau_w = wl[KMAX - 1];
            atomicMin(reinterpret_cast<unsigned long long *>(&s_tau), (unsigned long long)tau_w);
            wcount = KMAX;
        }
    };
    auto score = [&](const Chunk &ch) {
        int32_t vg[4];
        int32_t n12 = 0;
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
            // Rows 0..3 (registers 0..3 of row-0 lanes) hold sum (u/2) d_p: sum u Q = 2 sum_p 16^p D[p].
            const float dq = 2.f * (acc[0] + 16.f * (acc[1] + 16.f * (acc[2] + 16.f * acc[3])));
            vg[G] = (int32_t)dq;
            // Codes with u in {1, 2} of key 16G + col over this lane's 64 dims, summed over the 4 rows.
            int32_t p = 0;
#pragma unroll
            for (int s = 0; s < 4; s++) p += __popc((w[s] ^ (w[s] >> 1)) & 0x55555555u);
            p = rows_sum(p);
            n12 = row == G ? p : n12;
        }
        // Route group G's dot (valid in row 0) to row G: lane l ends with key l's.
        {
            auto a = __builtin_amdgcn_permlane32_swap((unsigned)vg[0], (unsigned)vg[2], false, false);
            auto b = __builtin_amdgcn_permlane32_swap((unsigned)vg[1], (unsigned)vg[3], false, false);
            auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
            vg[0] = (int32_t)c[0];
        }
        const int32_t duq = vg[0];
        const float sc = ch.sc;
        const int32_t dot = 2 * duq - 3 * sq;
        const int32_t c2 = c2_base - 8 * n12;
        const float t1 = (sc * sc) * 0.25f * (float)c2;
        const float t3 = (sc * qs) * (float)dot;
        const float dist = t1 - t3 + 0.0f;
        const uint64_t k64 = ((uint64_t)fkey(dist) << 32) | (uint64_t)(uint32_t)(ch.row0 + lane);
        const uint64_t ts = __hip_atomic_load(&s_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const uint64_t tau = tau_w < ts ? tau_w : ts;
        const bool take = lane < ch.nk && k64 < tau;
        const uint64_t mask = __ballot(take);
        if (take) {
            const int pos = wcount + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
            wl[pos] = k64;
        }
        wcount += __popcll(mask);
        if (wcount > CAPW - 64 || (tau_w == NONE && wcount >= 256)) wave_compact();
    };

    // (Both halves run unconditionally: a chunk past the end has nk = 0 and
    // scores nothing, and the loop body stays free of branches around loads.)
    // The empty asm with a memory clobber pins each fetch's loads above the
    // scoring that follows (the compiler would otherwise sink them to their
    // first use); nothing reads the loaded registers there, so no wait is added.
    Chunk ca, cb;
    if (nchunks > 0) {  // uniform over the workgroup
        // Phase A, in every wave: chunks wave and wave + 16 (2048 keys in all),
        // every key kept.  One workgroup sort then gives the exact 128th
        // smallest of them as the starting threshold of every wave; those 128
        // stay in fin[0..128).
        fetch(wave, ca);
        fetch(wave + SW, cb);
        asm volatile("" ::: "memory");
        score(ca);
        fetch(wave + 2 * SW, ca);
        asm volatile("" ::: "memory");
        score(cb);
        __syncthreads();
        for (int i = lane; i < wcount; i += 64) fin[atomicAdd(&count, 1)] = wl[i];
        __syncthreads();
        const int c0n = count;
        const int n0 = pow2_at_least(c0n);
        for (int i = c0n + tid; i < n0; i += STH) fin[i] = NONE;
        __syncthreads();
        bitonic_sort(fin, n0);
        if (tid == 0) {
            count = c0n < KMAX ? c0n : KMAX;
            if (c0n >= KMAX) s_tau = fin[KMAX - 1];
        }
        wcount = 0;
        __syncthreads();
        // Phase B: the rest, two chunks per trip.
        for (int32_t g = wave + 2 * SW; g < nchunks; g += 2 * SW) {
            fetch(g + SW, cb);
            asm volatile("" ::: "memory");
            score(ca);
            fetch(g + 2 * SW, ca);
            asm volatile("" ::: "memory");
            score(cb);
        }
    }
    // Final: every wave sorts its list and keeps its best 128; the keys at or
    // below the shared threshold (with the starting set, a superset of the
    // query's top 128) are gathered behind the starting set and sorted.
    wave_compact();
    __syncthreads();
    const uint64_t tfin = s_tau;
    for (int i = lane; i < wcount; i += 64) {
        const uint64_t e = wl[i];
        if (e <= tfin) fin[atomicAdd(&count, 1)] = e;
    }
    __syncthreads();
    const int cnt = count;
    const int n = pow2_at_least(cnt);
    for (int i = cnt + tid; i < n; i += STH) fin[i] = NONE;
    __syncthreads();
    bitonic_sort(fin, n);
    const float qn = s_qn;
    for (int j = tid; j < k; j += STH) {
        const uint64_t e = fin[j];
        if (e == NONE) {
            out_idx[q * k + j] = -1;
            out_dist[q * k + j] = __builtin_inff();
        } else {
            const float v = qn + unfkey((uint32_t)(e >> 32));
            out_idx[q * k + j] = (int64_t)(uint32_t)e;
            out_dist[q * k + j] = v > 0.f ? v : 0.f;
        }
    }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

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
    hipLaunchKernelGGL(k_search, dim3((unsigned)nq), dim3(STH), 0, st::stream_of(stream), codes, scales, cell_start,
                       ncells, queries, probes, (int32_t)nq, (int32_t)nprobe, (int32_t)k, out_idx, out_dist);
    ST_LAUNCH_CHECK();
    return ST_OK;
}
