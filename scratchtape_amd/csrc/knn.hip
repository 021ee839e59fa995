// 2-bit kNN memory on gfx950: device quantiser, fused dequant-dot scan with
// exact integer scoring, streaming per-(query, cell) top-128, per-query merge.
//
// Reference: gpu_step/knn.rs:190-225 (tile_of: the 2-bit quantiser),
// knn.rs:628-643 (k_dequant: code u decodes to (u - 1.5) * scale),
// gpu_step/knn/ivf.rs:194-321 (k_scan, k_dots_group), ivf.rs:466-686
// (search_ivf / scan_group), knn.rs:655-715 (merge of per-part lists) and the
// finalisation (dd + |q|^2).max(0) (ivf.rs:673-684).
//
// Scoring contract (replaces the reference's f16 x f16 -> f32 cmma dots, whose
// accumulation order no CPU can reproduce): the query is quantised to int16
// with a power-of-two scale qs, Q_i = clamp(rint(q_i / qs), +-32767), and with
// c_i = 2u_i - 3 the key decodes to c_i * s / 2.  Then
//     dot  = sum c_i Q_i        (exact, int32)
//     c2   = sum c_i^2          (exact, int32)
//     dist = ((s*s)*0.25f)*(float)c2 - (s*qs)*(float)dot
// with every f32 operation separately rounded (contraction off), which the CPU
// oracle reproduces bit for bit.  Ranking is by (dist, key index) ascending.
//
// Scan design: one 256-thread workgroup per (query, probed cell).  A wave
// reads 64 keys (4 KB of codes) per iteration as four fully coalesced 1 KB
// loads: lane l holds bytes 16*(l%4).. of key 16*s + l/4, i.e. 4 of the key's
// 16 code dwords, so each lane keeps only its quarter of the packed query (32
// VGPRs) and no LDS reads sit in the inner loop.  Per code dword:
// 4 masked shifts give bytes u in 0..3, one v_dot4_i32_i8 against the query's
// high bytes and one v_dot4_u32_u8 against its low bytes per shift, and one
// popcount for c2.  The four quarter-sums are combined with two butterfly
// shuffles (integer, so exact in any order).
//
// Top-k: candidates with key64 = (ordered dist bits << 32 | index) below the
// workgroup's threshold tau are appended to an LDS buffer of 1024; when it
// nears full, a bitonic sort keeps the 128 smallest and tau becomes the 128th.
// Only keys with at least 128 smaller keys already seen are ever dropped, so
// the cell's exact top-128 survives whatever the append order; the final sort
// makes the list deterministic.  A merge kernel sorts each query's nprobe lists
// and keeps the k best.
#include <cstring>

#include "common.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 256;          // key width handled by the scan
constexpr int DW = D / 16;      // code dwords per key
constexpr int KMAX = 128;       // neighbours kept per query (knn.rs:21)
constexpr int CAP = 1024;       // LDS candidate buffer (entries)
constexpr int PROBE_MAX = 16;   // most cells one query probes (ivf.rs:126)
constexpr int QPACK = 136;      // dwords per prepared query: 128 packed bytes + 4 scalars + pad
constexpr uint64_t NONE = ~0ull;

struct QScalars {
    float qs, qn;
    int32_t sq, pad;
};

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

// ---------------------------------------------------------------- query prep

// One wave per query: the int16 quantisation, then the bytes packed for the
// scan: dword (v, t, h) of code dword v holds, in byte j, the high (h = 0,
// signed) or low (h = 1, unsigned) byte of Q[16v + 4j + t], matching the
// bytes (w >> 2t) & 0x03030303 extracts from code dword v.
__global__ __launch_bounds__(64) void k_prep(const float *__restrict__ queries, uint32_t *__restrict__ qpack) {
    __shared__ uint8_t bytes[DW * 4 * 2 * 4];
    const int q = blockIdx.x, lane = threadIdx.x;
    const float4 v = reinterpret_cast<const float4 *>(queries + (int64_t)q * D)[lane];
    const float x[4] = {v.x, v.y, v.z, v.w};
    float mx = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float qs = 1.f, inv = 1.f;
    if (mx > 0.f) {
        int e;
        frexpf(mx, &e);
        qs = ldexpf(1.f, e - 15);
        inv = ldexpf(1.f, 15 - e);
    }
    int32_t sq = 0;
    double sq2 = 0.0;
    const int dwv = lane >> 2, j = lane & 3;  // dims 4*lane + t = 16*dwv + 4*j + t
#pragma unroll
    for (int t = 0; t < 4; t++) {
        float r = rintf(x[t] * inv);
        r = fminf(fmaxf(r, -32767.f), 32767.f);
        const int32_t Q = (int32_t)r;
        sq += Q;
        sq2 += (double)Q * (double)Q;
        bytes[((dwv * 4 + t) * 2 + 0) * 4 + j] = (uint8_t)((Q >> 8) & 0xff);
        bytes[((dwv * 4 + t) * 2 + 1) * 4 + j] = (uint8_t)(Q & 0xff);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        sq += __shfl_xor(sq, o, 64);
        sq2 += __shfl_xor(sq2, o, 64);
    }
    __syncthreads();
    uint32_t *dst = qpack + (int64_t)q * QPACK;
    dst[lane] = reinterpret_cast<const uint32_t *>(bytes)[lane];
    dst[lane + 64] = reinterpret_cast<const uint32_t *>(bytes)[lane + 64];
    if (lane == 0) {
        QScalars s;
        s.qs = qs;
        s.qn = (float)sq2 * (qs * qs);
        s.sq = sq;
        s.pad = 0;
        *reinterpret_cast<QScalars *>(dst + 128) = s;
    }
}

// ---------------------------------------------------------------- bitonic sort in LDS

// Sorts buf[0..n) ascending (n a power of two, <= 2048) with all 256 threads.
__device__ void bitonic_sort(uint64_t *buf, int n) {
    const int tid = threadIdx.x;
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < n; i += 256) {
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

__device__ __forceinline__ int pow2_at_least(int x) {
    int n = KMAX;
    while (n < x) n <<= 1;
    return n;
}

// ---------------------------------------------------------------- scan

__device__ __forceinline__ void quarter_dot(const uint4 &c, const uint32_t (&qh)[4][4], const uint32_t (&ql)[4][4],
                                            int32_t &hi, uint32_t &lo, uint32_t &n12) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int v = 0; v < 4; v++) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t e = (w[v] >> (2 * t)) & 0x03030303u;
            hi = __builtin_amdgcn_sdot4((int)e, (int)qh[v][t], hi, false);
            lo = __builtin_amdgcn_udot4(e, ql[v][t], lo, false);
        }
        n12 += __popc((w[v] ^ (w[v] >> 1)) & 0x55555555u);
    }
}

// grid: nq * nprobe workgroups of 256; workgroup (q, p) scans cell probes[q, p].
__global__ __launch_bounds__(256) void k_scan(const uint8_t *__restrict__ codes, const float *__restrict__ scales,
                                              const int64_t *__restrict__ cell_start, int64_t ncells,
                                              const int32_t *__restrict__ probes, int32_t nprobe,
                                              const uint32_t *__restrict__ qpack, uint64_t *__restrict__ lists) {
    __shared__ uint64_t cand[CAP];
    __shared__ int count;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t pair = blockIdx.x;
    const int64_t q = pair / nprobe;
    const int p = (int)(pair % nprobe);
    uint64_t *out = lists + pair * KMAX;

    const int32_t cell = probes[pair];
    bool skip = cell < 0 || cell >= ncells;
    for (int pp = 0; pp < p; pp++) skip |= probes[q * nprobe + pp] == cell;
    if (skip) {
        if (tid < KMAX) out[tid] = NONE;
        return;
    }
    const int64_t r0 = cell_start[cell], r1 = cell_start[cell + 1];

    // This lane's quarter of the packed query: code dwords 4*(lane%4) + v.
    const uint32_t *qp = qpack + q * QPACK;
    uint32_t qh[4][4], ql[4][4];
    const int quarter = lane & 3;
#pragma unroll
    for (int v = 0; v < 4; v++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            qh[v][t] = qp[((4 * quarter + v) * 4 + t) * 2 + 0];
            ql[v][t] = qp[((4 * quarter + v) * 4 + t) * 2 + 1];
        }
    const QScalars qsc = *reinterpret_cast<const QScalars *>(qp + 128);
    const int32_t c2_base = 9 * D;

    if (tid == 0) count = 0;
    uint64_t tau = NONE;
    __syncthreads();

    const uint4 *cbase = reinterpret_cast<const uint4 *>(codes);
    uint4 cur[4], nxt[4];
    auto load = [&](uint4 (&dst)[4], int64_t base) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int64_t key = base + wave * 64 + s * 16 + (lane >> 2);
            dst[s] = key < r1 ? cbase[key * 4 + quarter] : make_uint4(0, 0, 0, 0);
        }
    };
    load(cur, r0);
    for (int64_t base = r0; base < r1; base += 256) {
        if (base + 256 < r1) load(nxt, base + 256);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int64_t key = base + wave * 64 + s * 16 + (lane >> 2);
            int32_t hi = 0;
            uint32_t lo = 0, n12 = 0;
            quarter_dot(cur[s], qh, ql, hi, lo, n12);
            int32_t duq = hi * 256 + (int32_t)lo;
            duq += __shfl_xor(duq, 1, 64);
            duq += __shfl_xor(duq, 2, 64);
            n12 += __shfl_xor(n12, 1, 64);
            n12 += __shfl_xor(n12, 2, 64);
            if (quarter == 0 && key < r1) {
                const float sc = scales[key];
                const int32_t dot = 2 * duq - 3 * qsc.sq;
                const int32_t c2 = c2_base - 8 * (int32_t)n12;
                const float t1 = (sc * sc) * 0.25f * (float)c2;
                const float t3 = (sc * qsc.qs) * (float)dot;
                const float dist = t1 - t3 + 0.0f;
                const uint64_t k64 = ((uint64_t)fkey(dist) << 32) | (uint64_t)(uint32_t)key;
                if (k64 < tau) cand[atomicAdd(&count, 1)] = k64;
            }
        }
#pragma unroll
        for (int s = 0; s < 4; s++) cur[s] = nxt[s];
        __syncthreads();  // this iteration's appends are done
        const int cnt = count;
        __syncthreads();  // everyone has read count before the next appends
        if (cnt > CAP - 256) {
            const int n = pow2_at_least(cnt);
            for (int i = cnt + tid; i < n; i += 256) cand[i] = NONE;
            __syncthreads();
            bitonic_sort(cand, n);
            tau = cand[KMAX - 1];
            __syncthreads();
            if (tid == 0) count = KMAX;
            __syncthreads();
        }
    }
    const int cnt = count;
    const int n = pow2_at_least(cnt);
    for (int i = cnt + tid; i < n; i += 256) cand[i] = NONE;
    __syncthreads();
    bitonic_sort(cand, n);
    if (tid < KMAX) out[tid] = cand[tid];
}

// One workgroup per query: sort its nprobe lists, keep the k best, finalise.
__global__ __launch_bounds__(256) void k_merge(const uint64_t *__restrict__ lists, int32_t nprobe,
                                               const uint32_t *__restrict__ qpack, int32_t k,
                                               int64_t *__restrict__ out_idx, float *__restrict__ out_dist) {
    __shared__ uint64_t buf[PROBE_MAX * KMAX];
    const int64_t q = blockIdx.x;
    const int tid = threadIdx.x;
    const int total = nprobe * KMAX;
    int n = KMAX;
    while (n < total) n <<= 1;
    const uint64_t *src = lists + q * (int64_t)total;
    for (int i = tid; i < n; i += 256) buf[i] = i < total ? src[i] : NONE;
    __syncthreads();
    bitonic_sort(buf, n);
    const float qn = reinterpret_cast<const QScalars *>(qpack + q * QPACK + 128)->qn;
    for (int j = tid; j < k; j += 256) {
        const uint64_t e = buf[j];
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
    if (nq * nprobe > INT32_MAX) return st::fail(ST_ERR_INVALID, "search_ivf: too many queries for one call");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    const size_t qbytes = (size_t)nq * QPACK * 4;
    const size_t lbytes = (size_t)nq * nprobe * KMAX * 8;
    uint8_t *ws = static_cast<uint8_t *>(st::scratch(st::SCRATCH_KNN, qbytes + lbytes));
    if (!ws) return ST_ERR_OOM;
    uint32_t *qpack = reinterpret_cast<uint32_t *>(ws);
    uint64_t *lists = reinterpret_cast<uint64_t *>(ws + qbytes);
    hipStream_t s = st::stream_of(stream);
    hipLaunchKernelGGL(k_prep, dim3((unsigned)nq), dim3(64), 0, s, queries, qpack);
    ST_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_scan, dim3((unsigned)(nq * nprobe)), dim3(256), 0, s, codes, scales, cell_start, ncells,
                       probes, (int32_t)nprobe, qpack, lists);
    ST_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_merge, dim3((unsigned)nq), dim3(256), 0, s, lists, (int32_t)nprobe, qpack, (int32_t)k,
                       out_idx, out_dist);
    ST_LAUNCH_CHECK();
    return ST_OK;
}
