/*
 * scratchtape_hip.h — C ABI of the MI355X (gfx950) matrix-multiplication hot
 * path of scratchtape.  Every entry point is a drop-in for one reference
 * interface (cited per declaration, paths relative to the reference crate).
 *
 * Conventions
 *  - Device buffers are plain device pointers (the reference's cubecl
 *    `Handle`s).  The caller owns every operand and output; outputs are
 *    written in place.  The library owns only a grow-only scratch arena per
 *    device and use (split-k partials, probe-selection distances, LayerNorm
 *    column partials), like the reference's `split_scratch`
 *    (gpu_step/matmul.rs:207-217); the kNN search keeps its candidate lists
 *    in LDS and allocates nothing.  An arena grows only outside graph
 *    capture: a call that would grow it while its stream is being captured
 *    fails with ST_ERR_INVALID (run the call once before capturing).  A
 *    superseded arena buffer is kept, not freed, until st_scratch_release(),
 *    so a graph captured earlier never replays into freed memory.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL is the default
 *    stream) and is asynchronous, as the reference's single in-order queue
 *    (gpu_step/mod.rs:42, 78).  Calls that use the scratch arena (split-k
 *    GEMMs) must be serialised on one stream per device.
 *  - The reference panics (assert!/expect) on bad arguments.  Panics cannot
 *    cross an FFI boundary, so every entry point returns an st_status and
 *    st_last_error() gives the message (thread-local), whose text follows
 *    the reference's assert messages where one exists.
 */
#ifndef SCRATCHTAPE_HIP_H
#define SCRATCHTAPE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t st_status;
#define ST_OK 0
#define ST_ERR_INVALID (-1)     /* bad shape or argument (the reference's assert) */
#define ST_ERR_HIP (-2)         /* a HIP runtime call failed */
#define ST_ERR_OOM (-3)         /* scratch arena could not grow */
#define ST_ERR_NO_DEVICE (-4)   /* no gfx950 device visible */

typedef void *st_stream; /* hipStream_t */

/* A matrix inside a device buffer: gpu_step/matmul.rs:26-60 `MatRef`.
 * Matrix z starts at p + off + (z / group)*stride + (z % group)*inner; its
 * stored rows are `ld` apart (0: packed, the stored row length); `trans`: a
 * logical [r, c] operand stored as [c, r].  group 0 is read as 1. */
typedef struct st_matref {
    float *p;
    int64_t off;
    int64_t stride;
    int32_t trans;
    int32_t reserved;
    int64_t ld;
    int64_t group;
    int64_t inner;
} st_matref;

/* gpu_step/matmul.rs:62-79 `Epilogue`, applied in this order per output
 * element: + bias[bias_off + z*bias_stride + col], ReLU, zero where
 * mask[mask_off + (element index in out's layout)] <= 0, + residual (same
 * layout as out), + the value already in out (accumulate).  col_sum: also
 * add the column sums of b[z] over k into out.p[col_sum_off + z*col_sum_stride
 * + j] (always +=), summed in a fixed order.  NULL pointers mean "absent". */
typedef struct st_epilogue {
    const float *bias;
    int64_t bias_off;
    int64_t bias_stride;
    const float *mask;
    int64_t mask_off;
    const float *residual;
    int64_t residual_off;
    int32_t relu;
    int32_t accumulate;
    int32_t has_col_sum;
    int32_t reserved;
    int64_t col_sum_off;
    int64_t col_sum_stride;
} st_epilogue;

/* ---- GEMM: the three tape forms, batched, head views, epilogue ---------- */

/* gpu_step/matmul.rs:86 `matmul`: out[z] (+)= epi(a[z] @ b[z]) for z in
 * 0..batch, a[z] logically [m, k], b[z] [k, n], out row-major [m, n]
 * (out->trans must be 0: "out is stored row-major", matmul.rs:107).  Runs
 * f16-in/f32-accumulate when st_f16_enabled() and the shape tiles
 * (k % 32 == 0, m % 64 == 0, n % 32 == 0, and not col_sum with b
 * transposed: matmul.rs:108-112, 524-534), else f32.  epi may be NULL. */
st_status st_matmul(const st_matref *a, const st_matref *b, const st_matref *out, int64_t batch,
                    int64_t m, int64_t k, int64_t n, const st_epilogue *epi, st_stream stream);

/* gpu_step/matmul.rs:93 `matmul_f32`: the same, always f32 (the reference's
 * attention matmuls). */
st_status st_matmul_f32(const st_matref *a, const st_matref *b, const st_matref *out,
                        int64_t batch, int64_t m, int64_t k, int64_t n, const st_epilogue *epi,
                        st_stream stream);

/* gpu_step/matmul.rs:106 `matmul_with`: the f16 route chosen by the caller
 * (it still falls back to f32 for shapes it cannot tile). */
st_status st_matmul_with(const st_matref *a, const st_matref *b, const st_matref *out,
                         int64_t batch, int64_t m, int64_t k, int64_t n, const st_epilogue *epi,
                         int32_t use_f16, st_stream stream);

/* One GEMM of st_matmul_grouped: the arguments of st_matmul_with (an
 * all-zero epi is no epilogue). */
typedef struct st_gemm {
    st_matref a, b, out;
    st_epilogue epi;
    int64_t batch, m, k, n;
    int32_t use_f16;
    int32_t reserved;
} st_gemm;

/* GEMMs the reference issues back to back on its queue that do not depend on
 * each other, e.g. a Linear backward's dW = x^T dz (+ column sums) and
 * dx = dz W^T (gpu_step/tape.rs:324-347), as st_matmul_with each: no GEMM
 * of the group may read or write memory that another one writes.  Those that
 * tile by 128 x 128 (m % 128 == 0, n % 128 == 0, k % 32 == 0, k >= 128,
 * 16-byte aligned operands) run as one persistent launch per route (f16,
 * f32; up to 16 GEMMs per launch), the rest one by one.  Per element the
 * result equals st_matmul_with's, except that split-k may split k at other
 * points (the same fixed-order sum, other partial sums).  Uses the split-k
 * scratch arena: serialise on one stream per device. */
st_status st_matmul_grouped(const st_gemm *gemms, int64_t count, st_stream stream);

/* Size of the fixed device scratch of st_matmul_grouped_noalloc. */
#define ST_NOALLOC_SCRATCH_BYTES (64u << 20)

/* No counterpart in the reference: st_matmul_grouped for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results; the
 * split-k partials live in a fixed per-device array of
 * ST_NOALLOC_SCRATCH_BYTES instead of the library's arena, and the call
 * allocates and frees nothing.  A group whose partials need more is refused
 * with ST_ERR_INVALID before anything is launched (no output is touched).
 * Every call on a device shares that device's array: calls that overlap on
 * one device race. */
st_status st_matmul_grouped_noalloc(const st_gemm *gemms, int64_t count, st_stream stream);

/* gpu_step/matmul.rs:97-102 `f16_enabled`: 1 unless the environment sets
 * TRAIN_F16=0 (gfx950 always has f16 x f16 -> f32 matrix cores).  Read once. */
int32_t st_f16_enabled(void);

/* src/tensor.rs:241 `NdArray::matmul` on host buffers: out[m, n] = a[m, k] @
 * b[k, n], row-major f32, computed on the GPU in f32 (host buffers in and out;
 * synchronous).  Thread-safe: each call has its own stream and its own
 * split-k scratch (allocated and freed inside the call). */
st_status st_ndarray_matmul(const float *a, const float *b, float *out, int64_t m, int64_t k,
                            int64_t n);

/* ---- Row kernels of the attention configuration ------------------------ */

/* gpu_step/rows.rs:101-112 `softmax`: y = softmax(scale * x) per row of
 * x [rows, n].  causal: row r sees columns 0..=r % t, the rest are exactly
 * 0.  one: softmax1 (phantom logit 0, shift max(row max, 0)). */
st_status st_softmax(const float *x, float *y, int64_t rows, int64_t n, int64_t t, float scale,
                     int32_t causal, int32_t one, st_stream stream);

/* gpu_step/rows.rs:114-123 `softmax_backward`: dx = scale * y * (dy - sum(dy*y)). */
st_status st_softmax_backward(const float *dy, const float *y, float *dx, int64_t rows, int64_t n,
                              float scale, st_stream stream);

/* gpu_step/rows.rs:65 `layer_norm` (k_ln_fwd rows.rs:177-207; nn.rs:306-321):
 * y = (x - mean) / sqrt(var + eps) * gamma + beta per row of x [rows, d]
 * (biased variance); mean [rows] and rstd [rows] = 1 / sqrt(var + eps) are
 * kept for the backward.  gamma / beta are params[off + m stride + j] and
 * + d for the rows of model m (`Models`: rows split evenly over `models`
 * parameter sets `model_stride` floats apart; models = 1: stride unused). */
st_status st_layer_norm(const float *x, int64_t rows, int64_t d, const float *params, int64_t off,
                        float eps, int64_t models, int64_t model_stride, float *y, float *mean,
                        float *rstd, st_stream stream);

/* gpu_step/rows.rs:90 `layer_norm_backward` (k_ln_bwd_dx, k_ln_bwd_params
 * rows.rs:209-293): dx (+)= rstd (g - mean(g) - xhat mean(g xhat)), g = dy
 * gamma; grads[off + m stride + j] += sum of dy xhat over model m's rows,
 * grads[... + d + j] += sum of dy (always accumulated, in a fixed order).
 * Uses the library's row scratch arena (column partials): serialise on one
 * stream per device. */
st_status st_layer_norm_backward(const float *dy, const float *x, const float *mean,
                                 const float *rstd, int64_t rows, int64_t d, const float *params,
                                 float *grads, int64_t off, float *dx, int32_t accumulate,
                                 int64_t models, int64_t model_stride, st_stream stream);

/* ---- Fused causal attention ---------------------------------------------
 * The attention of the device tape (tape.rs:73-112; gpu_step/tape.rs:196-212,
 * 349-372: S = Q K^T, P = softmax(scale S) causal (rows.rs:101-112), O = P V
 * and their backward) in two launches that never write S or P.  Q, K, V are
 * the head-h column blocks [h hd, (h+1) hd) of the thirds of the fused QKV
 * buffer qkv [b t, 3 D] (D = h_count hd, window-major rows); ctx [b t, D] is O
 * in the merged layout; lse [b h_count t] the rows' log-sum-exp (max + log
 * sum, softmax1's phantom term included when one != 0), which the backward
 * uses to recompute P.  Operands are rounded to f16 (RNE) for f16 x f16 -> f32
 * matrix cores, as the f16 GEMM route rounds.  hd == 64, t a multiple of 32 in
 * 32..=256, 16-byte aligned buffers. */
st_status st_attention_fused_fwd(const float *qkv, float *ctx, float *lse, int64_t b, int64_t h,
                                 int64_t t, int64_t hd, float scale, int32_t one, st_stream stream);

/* Backward of st_attention_fused_fwd for the upstream gradient dctx [b t, D]:
 * writes dQ, dK, dV into the three blocks of dqkv [b t, 3 D] (every element;
 * rows.rs:114-123's dS = scale P (dP - rowsum(dP o P)), with rowsum(dP o P)
 * taken as rowsum(dO o O)). */
st_status st_attention_fused_bwd(const float *qkv, const float *ctx, const float *dctx,
                                 const float *lse, float *dqkv, int64_t b, int64_t h, int64_t t,
                                 int64_t hd, float scale, st_stream stream);

/* ---- 2-bit kNN memory ---------------------------------------------------- */

/* gpu_step/knn.rs:190-225 `tile_of` (bits = 2) on the device: keys [n, d]
 * f32 -> codes [n, d/4] (code i at byte i/4, bits 2(i%4)) and one f32 scale
 * per key, bit-identical to the reference's host quantiser.  d % 16 == 0. */
st_status st_knn_quantize_2bit(const float *keys, int64_t n, int64_t d, uint8_t *codes,
                               float *scales, st_stream stream);

/* gpu_step/knn.rs:216 (tile_of's norms): the per-key norm the reference
 * stores with a quantised tile (and its cache file, knn/cache.rs:49), the sum
 * over dims in order of f16((u - 1.5) * scale)^2 in f32; norms [n] device. */
st_status st_knn_key_norms_2bit(const uint8_t *codes, const float *scales, int64_t n, int64_t d,
                                float *norms, st_stream stream);

/* gpu_step/knn/ivf.rs:466 `KnnStore::search_ivf`, the scored part
 * (scan_group ivf.rs:528-686: fused dequant-dot, top-k, merge, finalise),
 * given each query's probed cells.  The store holds keys cell-contiguous:
 * cell c is rows cell_start[c]..cell_start[c+1] of codes [N, d/4] and
 * scales [N]; max_cell is the largest cell's row count (host-known from the
 * store build).  queries [nq, d] f32, probes [nq, nprobe] int32 cell ids (a
 * cell repeated within one query's probes is scanned once).  Outputs, per
 * query, the k (<= 128, KMAX knn.rs:21) nearest by the exact 2-bit score,
 * ascending by (distance, key index): out_idx [nq, k] global rows (-1
 * padding), out_dist [nq, k] = max(|q^|^2 + dist, 0) (+inf padding).
 * All pointers are device pointers; d == 256; the store holds fewer than
 * 2^32 keys (cell_start[ncells] < 2^32: key indices are 32-bit inside the
 * top-k keys).  A batch whose nq * nprobe probes reach 2/3 of ncells or
 * more (each cell probed 2/3 of a time or more on average; the reference
 * groups such batches by cell, ivf.rs:491-499) is scanned cell-major: each probed cell is read once
 * for up to four of its queries, with the per-pair lists in the library's
 * kNN scratch arena (nq * nprobe * 1 KiB; serialise such calls per device,
 * and run one before capturing a graph).  Smaller batches use no scratch. */
st_status st_knn_search_ivf_2bit(const uint8_t *codes, const float *scales,
                                 const int64_t *cell_start, int64_t ncells, int64_t max_cell,
                                 const float *queries, const int32_t *probes, int64_t nq,
                                 int64_t nprobe, int64_t d, int64_t k, int64_t *out_idx,
                                 float *out_dist, st_stream stream);

/* ---- IVF probe selection ---------------------------------------------------
 * Scoring contract: centroids and queries are quantised as the scan quantises
 * a query (int16 values X, power-of-two scale 2^e per vector, e = exponent of
 * max|x| - 14); dd = cnorm - ldexp(sum Q C, qe + ce + 1) in float64 with the
 * integer dot exact; cells ranked by (dd, cell id).  d == 256. */

/* No reference counterpart; for tests and benchmarks.  How
 * st_knn_search_ivf_2bit scans, process-wide, for calls enqueued afterwards:
 * 0 (default) chooses by batch size, 1 one workgroup per query (each probed
 * cell read once per query that probes it), 2 each probed cell read once for
 * up to four of the queries that probe it.  Both give identical results. */
st_status st_knn_set_scan_order(int32_t order);

/* Bytes of the digit store st_knn_centroids_prep writes for nlist centroids
 * (4096 per block of 8), or -1 for a width other than 256. */
int64_t st_knn_centroid_digit_bytes(int64_t nlist, int64_t d);

/* gpu_step/knn/ivf.rs:62-69 `Cent::new`: centroids [nlist, d] f32 (device) ->
 * digits (st_knn_centroid_digit_bytes bytes, 16-byte aligned; the quantised
 * centroids as int8 digit planes laid out for the matrix cores), cexp
 * [nlist] int32 scale exponents and cnorm [nlist] float64 squared norms of the
 * quantised centroids. */
st_status st_knn_centroids_prep(const float *centroids, int64_t nlist, int64_t d, int8_t *digits,
                                int32_t *cexp, double *cnorm, st_stream stream);

/* gpu_step/knn/ivf.rs:473-489 (the probe stage of `search_ivf`) and
 * ivf.rs:128-161 `k_probe`: for queries [nq, d] f32, probes [nq, nprobe]
 * int32 = each query's nprobe (1..=min(nlist, 16), PROBE_MAX ivf.rs:126)
 * nearest cells by (dd, cell id), nearest first.  digits/cexp/cnorm as
 * written by st_knn_centroids_prep.  Uses the library's kNN scratch arena
 * (float64 dd of up to 256 MiB per chunk of queries): calls that overlap on
 * one device race on it. */
st_status st_knn_probe(const int8_t *digits, const int32_t *cexp, const double *cnorm, int64_t nlist,
                       const float *queries, int64_t nq, int64_t d, int64_t nprobe, int32_t *probes,
                       st_stream stream);

/* gpu_step/knn.rs:295-331 `search_tagged` / `search_tail` (masked exact
 * search; key predicate of k_thresh / k_topk knn.rs:604-618) on the 2-bit
 * store of nkeys rows (KMAX <= nkeys < 2^31): query i scores the keys
 * g < always and lohi[2i] <= g < lohi[2i+1] (ranges clipped to the store;
 * lohi [nq, 2] int64 device) with the scoring and outputs of
 * st_knn_search_ivf_2bit (k nearest by (distance, key index), global key
 * rows, -1 / +inf padding).  The reference's from_key only skips tiles below
 * the ranges; scanning the two segments does that by construction. */
st_status st_knn_search_masked_2bit(const uint8_t *codes, const float *scales, int64_t nkeys,
                                    const float *queries, const int64_t *lohi, int64_t always,
                                    int64_t nq, int64_t d, int64_t k, int64_t *out_idx,
                                    float *out_dist, st_stream stream);

/* Benchmark support, no reference counterpart: fills rows [row0, row0 + n)
 * of a synthetic 2-bit store with keys drawn N(0,1) from a counter-based
 * generator (seed, global row, component) and quantised as
 * st_knn_quantize_2bit, without materialising the f32 keys.  d == 256. */
st_status st_knn_synth_store_2bit(uint64_t seed, int64_t row0, int64_t n, int64_t d,
                                  uint8_t *codes, float *scales, st_stream stream);

/* Benchmark/test support, no reference counterpart: the f32 keys [n, d] that
 * st_knn_synth_store_2bit quantises for rows [row0, row0 + n). */
st_status st_knn_synth_keys_f32(uint64_t seed, int64_t row0, int64_t n, int64_t d, float *keys,
                                st_stream stream);

/* ---- Device ceilings (benchmark support, no reference counterpart) ------- */

/* The current device's CU count, shader clock and memory clock (kHz) and
 * memory bus width (bits), from the HIP device attributes. */
st_status st_device_info(int32_t *cus, int32_t *clock_khz, int32_t *mem_clock_khz, int32_t *mem_bus_bits);

/* `blocks` workgroups of 4 waves, each wave running 8 independent MFMA chains
 * of `iters` steps: kind 0 v_mfma_f32_16x16x32_f16 (16384 FLOP per step),
 * 1 v_mfma_f32_16x16x4_f32 (2048), 2 v_mfma_i32_16x16x64_i8 (32768 OP),
 * 3 v_mfma_f32_32x32x16_f16 (32768), 4 v_mfma_i32_32x32x32_i8 (65536 OP).
 * The caller times it; `sink` ([blocks] floats) is never written in practice
 * (a guarded store keeps the chains live). */
st_status st_peak_mfma(int32_t kind, int64_t iters, int32_t blocks, float *sink, st_stream stream);

/* Reads `bytes` (a multiple of 16, 16-byte aligned) of src once with `blocks`
 * workgroups of 256 threads, each streaming its own contiguous slab with
 * nontemporal loads; `sink` as for st_peak_mfma. */
st_status st_peak_read(const void *src, int64_t bytes, int32_t blocks, float *sink, st_stream stream);

/* Checks the cross-lane exchanges the kernels use (DPP and v_permlane swaps in
 * place of ds_bpermute) on the current device: `out` (device, 10 x 64
 * uint32) gets, for one wave, rows 0..7 the exchange of v = 1000 + 7 lane
 * across lane ^ J for J = 1, 2, 4, 8, 15, 16, 32, 63 (expected 1000 + 7
 * (lane ^ J)), row 8 the inclusive wave scan of 3 lane + 1 + lane % 5, row 9
 * lane 37's v in every lane. */
st_status st_lane_selftest(uint32_t *out, st_stream stream);

/* ---- Misc ---------------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char *st_last_error(void);

/* No reference counterpart (the reference's cubecl client owns its memory
 * until exit): waits for every device the library used, then frees all of its
 * scratch arenas, current and superseded.  Only for callers that will not
 * replay again any graph that captured a library call; the next call that
 * needs scratch allocates it anew.  It must not run concurrently with any
 * other library call (another thread's call may hold an arena buffer it has
 * not yet launched into). */
st_status st_scratch_release(void);

/* Waits for the work enqueued on `stream`.  It then also checks the current
 * device for slot waits of the grouped f16 GEMM kernel that gave up (each
 * wait is bounded so that the kernel always ends; a give-up means its
 * producer and consumer waves lost step, and the outputs of the grouped f16
 * GEMMs run since the last check are not valid): ST_ERR_HIP with a message
 * if there were any, and the count is cleared.  Reference failures surface
 * as panics (tensor.rs:253, gpu_step/matmul.rs:107). */
st_status st_sync(st_stream stream);

/* No reference counterpart; for tests of the check above.  Sets how many
 * times a slot wait of the grouped f16 GEMM kernel polls its counter before
 * it gives up, for launches enqueued afterwards (process-wide; a negative
 * value restores the default, 2^20). */
st_status st_set_wait_limit(int64_t polls);

/* Library version string. */
const char *st_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SCRATCHTAPE_HIP_H */
