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
// Design.  The int16 values are split into two int8 digits, X = 256 Xh + Xl
// with Xl in [-128, 127] and Xh in [-64, 64], so one i8 MFMA
// (16 x 16 x 64, int32 accumulate) yields all four digit products of 8
// queries x 8 centroids over 64 dims: A rows are (query, digit), B columns
// (centroid, digit), and dot = 65536 hh + 256 (hl + lh) + ll is assembled
// from two neighbouring lanes.  Digits are stored "MFMA-native": a block of
// 8 vectors is 4 KiB, [k-step s][lane][16 bytes], so each operand load is one
// fully coalesced 1 KiB read.  Three kernels:
//   k_probe_prep   vectors -> digit blocks, exponent (and norm for centroids);
//   k_probe_dots   dd for a chunk of queries x every centroid (float64, in the
//                  library's scratch arena);
//   k_probe_select one workgroup per query: a threshold from the per-thread
//                  minima keeps about nprobe candidates per round of cells,
//                  which one wave sorts by (dd, id).
#include "common.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 256;              // vector width (the scan's key width)
constexpr int BLK = 8;              // vectors per digit block
constexpr int BLK_BYTES = BLK * 2 * D;  // 4096
constexpr int PROBE_MAX = 16;       // ivf.rs:126
constexpr int PER_MAX = 8;          // centroid blocks per dots workgroup (staged in LDS)
constexpr int64_t DD_BUDGET = 256ll << 20;  // bytes of dd per query chunk

typedef int32_t v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// One wave per vector (row r of x [n, D]); lane L handles dims 4L .. 4L + 3.
// Writes the vector's two digit planes into its block (rows n .. of the last
// block are zero), its exponent, and, when norm != nullptr, its squared norm.
// Byte (s, lane, j) of a block is dim 64 s + 16 (lane / 16) + j of vector
// (lane % 16) / 2, digit lane % 2 (0: high, 1: low).
__global__ __launch_bounds__(256) void k_probe_prep(const float *__restrict__ x, int64_t n, int8_t *__restrict__ dig,
                                                    int32_t *__restrict__ ex, double *__restrict__ norm) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t nblk = (n + BLK - 1) / BLK;
    if (r >= nblk * BLK) return;
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
        // ldexpf is exact here (|result| < 2^14), and equals x / 2^(e-14).
        const int32_t X = (int32_t)fminf(fmaxf(rintf(ldexpf(v[t], 14 - e)), -16384.f), 16383.f);
        const int32_t xl = ((X + 128) & 255) - 128;
        const int32_t xh = (X - xl) >> 8;
        lo |= (uint32_t)(xl & 255) << (8 * t);
        hi |= (uint32_t)(xh & 255) << (8 * t);
        s2 += X * X;
    }
    const int v8 = (int)(r % BLK);
    const int s = lane >> 4, g = (lane & 15) >> 2, j0 = 4 * (lane & 3);
    int8_t *blk = dig + (r / BLK) * BLK_BYTES + s * 1024 + j0;
    *reinterpret_cast<uint32_t *>(blk + (16 * g + 2 * v8) * 16) = hi;
    *reinterpret_cast<uint32_t *>(blk + (16 * g + 2 * v8 + 1) * 16) = lo;
    if (r >= n) return;
    if (norm) {
        double t2 = (double)s2;  // partial sums are integers below 2^53: exact in any order
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) t2 += __shfl_xor(t2, o, 64);
        if (lane == 0) norm[r] = ldexp(t2, 2 * (e - 14));
    }
    if (lane == 0) ex[r] = e - 14;
}

// dd[q][c] for queries [q0, q0 + nqc) of the chunk (digit blocks qdig, exponents
// qex, chunk-relative) against centroids [0, nlist).  grid.y: groups of 8 query
// blocks (wave w takes blocks 8 y + 2 w and + 1); grid.x: slices of `per`
// (<= PER_MAX) centroid blocks, which the workgroup stages in LDS (digits,
// norms, exponents: every load in flight at once) before its waves walk them.
__global__ __launch_bounds__(256) void k_probe_dots(const int8_t *__restrict__ qdig, const int32_t *__restrict__ qex,
                                                    int32_t nqc, const int8_t *__restrict__ cdig,
                                                    const int32_t *__restrict__ cexp, const double *__restrict__ cnorm,
                                                    int32_t nlist, int32_t per, double *__restrict__ dd) {
    __shared__ v4i s_dig[PER_MAX * BLK_BYTES / 16];
    __shared__ double s_cn[PER_MAX * BLK];
    __shared__ int32_t s_ce[PER_MAX * BLK];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nqb = (nqc + BLK - 1) / BLK;
    const int qb0 = blockIdx.y * 8 + 2 * w;
    const bool active = qb0 < nqb, two = qb0 + 1 < nqb;
    const int ncb = (nlist + BLK - 1) / BLK;
    const int cb0 = blockIdx.x * per;
    const int cb1 = min(cb0 + per, ncb);

    v4i a[2][4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        a[0][s] = active ? *reinterpret_cast<const v4i *>(qdig + (int64_t)qb0 * BLK_BYTES + s * 1024 + lane * 16)
                         : v4i{0, 0, 0, 0};
        a[1][s] = two ? *reinterpret_cast<const v4i *>(qdig + (int64_t)(qb0 + 1) * BLK_BYTES + s * 1024 + lane * 16)
                      : v4i{0, 0, 0, 0};
    }
    {
        const int nb = cb1 - cb0;
        const v4i *src = reinterpret_cast<const v4i *>(cdig + (int64_t)cb0 * BLK_BYTES);
#pragma unroll
        for (int i = 0; i < PER_MAX; i++)
            if (i < nb) s_dig[i * 256 + threadIdx.x] = src[i * 256 + threadIdx.x];
        if (threadIdx.x < nb * BLK) {
            const int c = cb0 * BLK + threadIdx.x;
            s_cn[threadIdx.x] = c < nlist ? cnorm[c] : 0.0;
            s_ce[threadIdx.x] = c < nlist ? cexp[c] : 0;
        }
    }
    __syncthreads();
    if (!active) return;
    const bool odd = lane & 1;
    const int qv = 2 * (lane >> 4) + (lane & 1);  // query within a block
    const int cv = (lane & 15) >> 1;              // centroid within a block
    int qe[2];
    bool qok[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int qi = (qb0 + u) * BLK + qv;
        qok[u] = qi < nqc;
        qe[u] = qok[u] ? qex[qi] : 0;
    }

#pragma unroll 1
    for (int cb = cb0; cb < cb1; cb++) {
        const int k = cb - cb0;
        v4i b[4];
#pragma unroll
        for (int s = 0; s < 4; s++) b[s] = s_dig[k * 256 + s * 64 + lane];
        const double cn = s_cn[k * BLK + cv];
        const int ce = s_ce[k * BLK + cv];
        v4i acc[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            acc[u] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < 4; s++) acc[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u][s], b[s], acc[u], 0, 0, 0);
        }
        const int c = cb * BLK + cv;
        const bool cok = c < nlist;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            // Lane l holds rows 4 (l/16) .. + 3 (queries 2 (l/16) and + 1, digits
            // high, low) of column l % 16 (centroid (l%16)/2, digit l % 2).  An
            // even lane assembles query 2 (l/16), an odd lane query 2 (l/16) + 1.
            const int32_t s0 = odd ? acc[u][0] : acc[u][2];
            const int32_t s1 = odd ? acc[u][1] : acc[u][3];
            const int32_t r0 = __shfl_xor(s0, 1, 64), r1 = __shfl_xor(s1, 1, 64);
            const int32_t hh = odd ? r0 : acc[u][0];
            const int32_t lh = odd ? r1 : acc[u][1];
            const int32_t hl = odd ? acc[u][2] : r0;
            const int32_t ll = odd ? acc[u][3] : r1;
            const int64_t dot = (int64_t)hh * 65536 + (int64_t)(hl + lh) * 256 + ll;
            if (cok && qok[u]) {
                const int64_t qi = (int64_t)(qb0 + u) * BLK + qv;
                dd[qi * nlist + c] = cn - ldexp((double)dot, qe[u] + ce + 1);
            }
        }
    }
}

// Order-preserving map of a float64 onto u64 (finite values; -0 < +0).
__device__ __forceinline__ uint64_t dkey(double v) {
    const uint64_t x = (uint64_t)__double_as_longlong(v);
    return (x >> 63) ? ~x : (x | (1ull << 63));
}

__device__ __forceinline__ bool lt(uint64_t ka, int32_t ia, uint64_t kb, int32_t ib) {
    return ka < kb || (ka == kb && ia < ib);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m, 64), hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

// Wave-wide minimum of (key, id); every lane receives it.
__device__ __forceinline__ void wave_min(uint64_t &k, int32_t &i) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t ko = shfl_xor_u64(k, o);
        const int32_t io = __shfl_xor(i, o, 64);
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
            const uint32_t y = __shfl_xor(x, j, 64);
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
            const int32_t io = __shfl_xor(i, j, 64);
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
constexpr int SEL_T = 1024;         // threads per query
constexpr int SEL_W = SEL_T / 64;   // waves
constexpr int SEL_J = 12;           // cells per thread and round
constexpr int SEL_ROUND = SEL_T * SEL_J;
constexpr int CAND = 1024;          // LDS candidate buffer

// One workgroup of 1024 threads per query q of the chunk: probes[q][0, nprobe)
// by (dd, id) ascending.  Rounds of 12288 cells: every thread loads its 12
// values at once; a threshold on the high 32 bits of the ordered keys is the
// nprobe-th smallest of the 1024 per-thread minima (so at least nprobe
// candidates lie at or below it, and every member of the top nprobe does);
// the candidates at or below it (about nprobe of them) and the running top
// nprobe are collected in LDS and sorted by one wave.  Should the buffer
// overflow (many equal distances), the round is re-read from memory by
// nprobe successive minimum searches instead, which is exact for any input.
__global__ __launch_bounds__(SEL_T) void k_probe_select(const double *__restrict__ dd, int32_t nlist, int32_t nprobe,
                                                        int32_t *__restrict__ probes) {
    __shared__ uint64_t s_ck[CAND];
    __shared__ int32_t s_ci[CAND];
    __shared__ uint32_t s_lm[SEL_W][PROBE_MAX];
    __shared__ uint64_t s_bk[PROBE_MAX];
    __shared__ int32_t s_bi[PROBE_MAX];
    __shared__ uint32_t s_tau;
    __shared__ int32_t s_cnt, s_nb;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t q = blockIdx.x;
    const double *row = dd + q * nlist;
    if (tid == 0) s_nb = 0;

    for (int base = 0; base < nlist; base += SEL_ROUND) {
        uint64_t key[SEL_J];
#pragma unroll
        for (int j = 0; j < SEL_J; j++) {
            const int c = base + j * SEL_T + tid;
            key[j] = c < nlist ? dkey(row[c]) : KNONE;
        }
        uint32_t m = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < SEL_J; j++) m = min(m, (uint32_t)(key[j] >> 32));
        const uint32_t ms = wave_sort_u32(m, lane);
        if (lane < nprobe) s_lm[w][lane] = ms;
        __syncthreads();  // also orders the previous round's s_bk / s_nb before their use below
        if (w == 0) {
            // nprobe-th smallest of the 16 waves' nprobe smallest minima (the
            // nprobe-th smallest of all 1024), and the running top's bound.
            uint32_t v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int e = r * 64 + lane;
                v[r] = e < SEL_W * nprobe ? s_lm[e / nprobe][e % nprobe] : 0xffffffffu;
            }
            uint32_t t = 0xffffffffu;
            for (int r = 0; r < nprobe; r++) {
                uint32_t lm = min(min(v[0], v[1]), min(v[2], v[3]));
                uint32_t wm = lm;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) wm = min(wm, __shfl_xor(wm, o, 64));
                t = wm;
                // The lowest lane holding wm drops one copy of it.
                const uint64_t holders = __ballot(lm == wm);
                if (lane == __builtin_ctzll(holders)) {
                    if (v[0] == wm) v[0] = 0xffffffffu;
                    else if (v[1] == wm) v[1] = 0xffffffffu;
                    else if (v[2] == wm) v[2] = 0xffffffffu;
                    else v[3] = 0xffffffffu;
                }
            }
            const int nb = s_nb;
            if (nb == nprobe) t = min(t, (uint32_t)(s_bk[nprobe - 1] >> 32));
            if (lane == 0) {
                s_tau = t;
                s_cnt = nb;
            }
            if (lane < nb) {  // the running top nprobe are candidates too
                s_ck[lane] = s_bk[lane];
                s_ci[lane] = s_bi[lane];
            }
        }
        __syncthreads();
        const uint32_t tau = s_tau;
        int npass = 0;
#pragma unroll
        for (int j = 0; j < SEL_J; j++) npass += __popcll(__ballot((uint32_t)(key[j] >> 32) <= tau && key[j] != KNONE));
        int off = 0;
        if (lane == 0 && npass) off = atomicAdd(&s_cnt, npass);
        off = __shfl(off, 0, 64);
#pragma unroll
        for (int j = 0; j < SEL_J; j++) {
            const bool pass = (uint32_t)(key[j] >> 32) <= tau && key[j] != KNONE;
            const uint64_t bal = __ballot(pass);
            const int pos = off + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
            if (pass && pos < CAND) {
                s_ck[pos] = key[j];
                s_ci[pos] = base + j * SEL_T + tid;
            }
            off += __popcll(bal);
        }
        __syncthreads();
        if (w == 0) {
            const int cnt = s_cnt;
            int nb = 0;
            if (cnt <= 64) {
                uint64_t k = lane < cnt ? s_ck[lane] : KNONE;
                int32_t i = lane < cnt ? s_ci[lane] : INONE;
                wave_sort_pair(k, i, lane);
                nb = min(cnt, nprobe);
                if (lane < nb) {
                    s_bk[lane] = k;
                    s_bi[lane] = i;
                }
            } else {
                // nprobe successive minima strictly above the last one taken
                // (the pairs are distinct): over the buffer, or, if it
                // overflowed, over the round's cells and the running top.
                const bool over = cnt > CAND;
                const int nbo = s_nb;
                const uint64_t tk = lane < nbo ? s_bk[lane] : KNONE;  // the running top, read before it is replaced
                const int32_t ti = lane < nbo ? s_bi[lane] : INONE;
                uint64_t lk = 0, rk = KNONE;
                int32_t li = -1, ri = INONE;
                const int end = min(nlist - base, SEL_ROUND);
                for (int r = 0; r < nprobe; r++) {
                    uint64_t bk = KNONE;
                    int32_t bi = INONE;
                    if (!over) {
                        for (int e = lane; e < cnt; e += 64) {
                            const uint64_t k = s_ck[e];
                            const int32_t i = s_ci[e];
                            if (lt(lk, li, k, i) && lt(k, i, bk, bi)) {
                                bk = k;
                                bi = i;
                            }
                        }
                    } else {
                        for (int e = lane; e < end; e += 64) {
                            const uint64_t k = dkey(row[base + e]);
                            const int32_t i = base + e;
                            if (lt(lk, li, k, i) && lt(k, i, bk, bi)) {
                                bk = k;
                                bi = i;
                            }
                        }
                        if (lt(lk, li, tk, ti) && lt(tk, ti, bk, bi)) {
                            bk = tk;
                            bi = ti;
                        }
                    }
                    wave_min(bk, bi);
                    if (bk == KNONE && bi == INONE) break;
                    if (lane == r) {
                        rk = bk;
                        ri = bi;
                    }
                    lk = bk;
                    li = bi;
                    nb = r + 1;
                }
                if (lane < nb) {
                    s_bk[lane] = rk;
                    s_bi[lane] = ri;
                }
            }
            if (lane == 0) s_nb = nb;
        }
    }
    __syncthreads();
    if (tid < nprobe) probes[q * nprobe + tid] = tid < s_nb ? s_bi[tid] : -1;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

st_status launch_prep(const float *x, int64_t n, int8_t *dig, int32_t *ex, double *norm, hipStream_t s) {
    const int64_t rows = cdiv(n, BLK) * BLK;
    hipLaunchKernelGGL(k_probe_prep, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, x, n, dig, ex, norm);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

}  // namespace

extern "C" int64_t st_knn_centroid_digit_bytes(int64_t nlist, int64_t d) {
    if (nlist < 0 || d != D) return -1;
    return cdiv(nlist, BLK) * BLK_BYTES;
}

extern "C" st_status st_knn_centroids_prep(const float *centroids, int64_t nlist, int64_t d, int8_t *digits,
                                           int32_t *cexp, double *cnorm, st_stream stream) {
    st::clear_error();
    if (!centroids || !digits || !cexp || !cnorm) return st::fail(ST_ERR_INVALID, "centroids_prep: NULL buffer");
    if (d != D) return st::fail(ST_ERR_INVALID, "centroids_prep: built for d == %d (got %lld)", D, (long long)d);
    if (nlist < 1 || nlist > INT32_MAX - BLK)
        return st::fail(ST_ERR_INVALID, "centroids_prep: nlist must be in 1..2^31 - 9 (got %lld)", (long long)nlist);
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
    if (nlist < 1 || nlist > INT32_MAX - BLK || nq < 0)
        return st::fail(ST_ERR_INVALID, "probe: bad nlist or nq");
    if (nprobe < 1 || nprobe > nlist || nprobe > PROBE_MAX)
        return st::fail(ST_ERR_INVALID, "probe: nprobe must be in 1..=min(nlist, %d) (got %lld)", PROBE_MAX,
                        (long long)nprobe);
    if ((reinterpret_cast<uintptr_t>(queries) & 15) != 0 || (reinterpret_cast<uintptr_t>(digits) & 15) != 0)
        return st::fail(ST_ERR_INVALID, "probe: queries and digits must be 16-byte aligned");
    if (nq == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const hipStream_t s = st::stream_of(stream);

    // Queries in chunks whose dd matrix fits DD_BUDGET (multiples of 64 queries).
    int64_t chunk = DD_BUDGET / (nlist * (int64_t)sizeof(double));
    chunk = chunk < 64 ? 64 : chunk / 64 * 64;
    if (chunk > nq) chunk = cdiv(nq, BLK) * BLK;
    const int64_t dd_bytes = chunk * nlist * (int64_t)sizeof(double);
    const int64_t dig_bytes = cdiv(chunk, BLK) * BLK_BYTES;
    char *base = static_cast<char *>(st::scratch(st::SCRATCH_KNN, (size_t)(dd_bytes + dig_bytes + chunk * 4), s));
    if (!base) return st::scratch_status();
    double *dd = reinterpret_cast<double *>(base);
    int8_t *qdig = reinterpret_cast<int8_t *>(base + dd_bytes);
    int32_t *qex = reinterpret_cast<int32_t *>(base + dd_bytes + dig_bytes);

    const int64_t ncb = cdiv(nlist, BLK);
    for (int64_t q0 = 0; q0 < nq; q0 += chunk) {
        const int64_t nqc = nq - q0 < chunk ? nq - q0 : chunk;
        st_status st = launch_prep(queries + q0 * D, nqc, qdig, qex, nullptr, s);
        if (st != ST_OK) return st;
        const int64_t gy = cdiv(cdiv(nqc, BLK), 8);
        int64_t per = cdiv(ncb * gy, 1024);
        if (per < 2) per = 2;
        if (per > PER_MAX) per = PER_MAX;
        const int64_t gx = cdiv(ncb, per);
        hipLaunchKernelGGL(k_probe_dots, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, s, qdig, qex, (int32_t)nqc,
                           digits, cexp, cnorm, (int32_t)nlist, (int32_t)per, dd);
        ST_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_probe_select, dim3((unsigned)nqc), dim3(SEL_T), 0, s, dd, (int32_t)nlist, (int32_t)nprobe,
                           probes + q0 * nprobe);
        ST_LAUNCH_CHECK();
    }
    return ST_OK;
}
