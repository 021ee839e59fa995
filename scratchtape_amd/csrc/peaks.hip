// Device ceilings for the benchmark's roofline context (no reference
// counterpart, on no data path): the matrix cores' throughput with nothing but
// independent MFMA chains in flight, the HBM read rate of a plain streaming
// kernel in the key scans' launch shape, and the device's CU count and clocks.  The benchmark reports these
// beside the published peaks it prices every kernel against.
#include "common.h"
#include "lanes.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

constexpr int CHAINS = 8;  // independent accumulators per wave (covers the MFMA latency)

// Never true for the values these kernels accumulate; the guarded store keeps
// every chain's result live without writing memory.
constexpr float NEVER = -1.2345e30f;

// kind 0: v_mfma_f32_16x16x32_f16, 1: v_mfma_f32_16x16x4_f32,
// 2: v_mfma_i32_16x16x64_i8, 3: v_mfma_f32_32x32x16_f16 (the GEMMs' form),
// 4: v_mfma_i32_32x32x32_i8.  Operands come from the lane id so that nothing
// folds; magnitudes stay small, so no accumulator overflows or turns inf.
template <int KIND>
__global__ __launch_bounds__(256) void k_peak_mfma(int64_t iters, float *__restrict__ sink) {
    const int lane = threadIdx.x & 63;
    float s = 0.f;
    if constexpr (KIND == 0) {
        half8 a, b;
        for (int e = 0; e < 8; e++) {
            a[e] = (_Float16)(1e-3f * (float)((lane + e) & 7));
            b[e] = (_Float16)(1e-3f * (float)((lane * 3 + e) & 7));
        }
        f32x4 acc[CHAINS];
        for (int c = 0; c < CHAINS; c++) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int64_t i = 0; i < iters; i++) {
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
        }
        for (int c = 0; c < CHAINS; c++) s += acc[c][0] + acc[c][3];
    } else if constexpr (KIND == 1) {
        const float a = 1e-3f * (float)(lane & 7), b = 1e-3f * (float)((lane * 3) & 7);
        f32x4 acc[CHAINS];
        for (int c = 0; c < CHAINS; c++) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int64_t i = 0; i < iters; i++) {
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c], 0, 0, 0);
        }
        for (int c = 0; c < CHAINS; c++) s += acc[c][0] + acc[c][3];
    } else if constexpr (KIND == 3) {
        half8 a, b;
        for (int e = 0; e < 8; e++) {
            a[e] = (_Float16)(1e-3f * (float)((lane + e) & 7));
            b[e] = (_Float16)(1e-3f * (float)((lane * 3 + e) & 7));
        }
        f32x16 acc[CHAINS];
        for (int c = 0; c < CHAINS; c++)
            for (int e = 0; e < 16; e++) acc[c][e] = 0.f;
        for (int64_t i = 0; i < iters; i++) {
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
        }
        for (int c = 0; c < CHAINS; c++) s += acc[c][0] + acc[c][15];
    } else if constexpr (KIND == 4) {
        const v4i a = {lane & 1, (lane >> 1) & 1, 0, 1}, b = {1, 0, lane & 1, 0};
        v16i acc[CHAINS];
        for (int c = 0; c < CHAINS; c++)
            for (int e = 0; e < 16; e++) acc[c][e] = 0;
        for (int64_t i = 0; i < iters; i++) {
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
        }
        for (int c = 0; c < CHAINS; c++) s += (float)(acc[c][0] + acc[c][15]);
    } else {
        const v4i a = {lane & 1, (lane >> 1) & 1, 0, 1}, b = {1, 0, lane & 1, 0};
        v4i acc[CHAINS];
        for (int c = 0; c < CHAINS; c++) acc[c] = v4i{0, 0, 0, 0};
        for (int64_t i = 0; i < iters; i++) {
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
        }
        for (int c = 0; c < CHAINS; c++) s += (float)(acc[c][0] + acc[c][3]);
    }
    if (s == NEVER) sink[blockIdx.x] = s;
}

// Reads src [n4] float4 once with nontemporal (streaming) loads: workgroup b
// reads its own contiguous slab (whole 1 KB blocks), its 4 waves taking the
// slab's 1 KB blocks in turn, each lane with sixteen 16-byte loads in flight.
// With eight such workgroups per CU this is the fastest read shape measured on
// the device (about 7.0 TB/s; 256 workgroups of 16 waves with allocating loads
// and eight in flight: about 5.9).
constexpr int RT = 256;       // threads per workgroup
constexpr int RDEPTH = 16;    // loads in flight per lane
typedef float v4f_nt __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(RT) void k_peak_read(const float4 *__restrict__ src, int64_t n4,
                                                  float *__restrict__ sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t per = ((n4 + gridDim.x - 1) / gridDim.x + 63) / 64 * 64;
    const int64_t s0 = (int64_t)blockIdx.x * per;
    const int64_t s1 = s0 + per < n4 ? s0 + per : n4;
    constexpr int64_t STEP = (int64_t)RDEPTH * (RT / 64) * 64;
    float acc = 0.f;
    for (int64_t b = s0 + (int64_t)wave * 64 + lane; b < s1; b += STEP) {
        float4 v[RDEPTH];
#pragma unroll
        for (int d = 0; d < RDEPTH; d++) {
            const int64_t e = b + (int64_t)d * (RT / 64) * 64;
            if (e < s1) {
                const v4f_nt t = __builtin_nontemporal_load(reinterpret_cast<const v4f_nt *>(src) + e);
                v[d] = float4{t.x, t.y, t.z, t.w};
            } else {
                v[d] = float4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int d = 0; d < RDEPTH; d++) acc += v[d].x + v[d].w;
    }
    if (acc == NEVER) sink[blockIdx.x] = acc;
}

// One wave: row r < 8 of out gets xor_lane(1000 + 7 lane, J[r], lane) for
// J = 1, 2, 4, 8, 15, 16, 32, 63 (lane ^ J's value, 1000 + 7 (lane ^ J));
// row 8 the inclusive wave scan of 3 lane + 1 + lane % 5; row 9 lane 37's
// value broadcast by lane_value.
__global__ __launch_bounds__(64) void k_lane_selftest(uint32_t *__restrict__ out) {
    const int lane = threadIdx.x;
    const uint32_t v = 1000u + 7u * (uint32_t)lane;
    constexpr int J[8] = {1, 2, 4, 8, 15, 16, 32, 63};
#pragma unroll
    for (int r = 0; r < 8; r++) out[r * 64 + lane] = st::xor_lane(v, J[r], lane);
    out[8 * 64 + lane] = (uint32_t)st::wave_incl_scan(3 * lane + 1 + lane % 5);
    out[9 * 64 + lane] = st::lane_value(v, 37);
}

}  // namespace

extern "C" st_status st_device_info(int32_t *cus, int32_t *clock_khz, int32_t *mem_clock_khz,
                                    int32_t *mem_bus_bits) {
    st::clear_error();
    if (!cus || !clock_khz || !mem_clock_khz || !mem_bus_bits) return st::fail(ST_ERR_INVALID, "device_info: NULL");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    int dev = 0;
    ST_HIP_CHECK(hipGetDevice(&dev));
    ST_HIP_CHECK(hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev));
    ST_HIP_CHECK(hipDeviceGetAttribute(clock_khz, hipDeviceAttributeClockRate, dev));
    ST_HIP_CHECK(hipDeviceGetAttribute(mem_clock_khz, hipDeviceAttributeMemoryClockRate, dev));
    ST_HIP_CHECK(hipDeviceGetAttribute(mem_bus_bits, hipDeviceAttributeMemoryBusWidth, dev));
    return ST_OK;
}

extern "C" st_status st_peak_mfma(int32_t kind, int64_t iters, int32_t blocks, float *sink, st_stream stream) {
    st::clear_error();
    if (kind < 0 || kind > 4)
        return st::fail(ST_ERR_INVALID,
                        "peak_mfma: kind is 0 (f16 16x16x32), 1 (f32), 2 (i8 16x16x64), 3 (f16 32x32x16) or 4 (i8 "
                        "32x32x32)");
    if (iters < 1 || blocks < 1 || !sink) return st::fail(ST_ERR_INVALID, "peak_mfma: bad iters, blocks or sink");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    void (*const kernels[])(int64_t, float *) = {k_peak_mfma<0>, k_peak_mfma<1>, k_peak_mfma<2>, k_peak_mfma<3>,
                                                  k_peak_mfma<4>};
    void (*k)(int64_t, float *) = kernels[kind];
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(256), 0, st::stream_of(stream), iters, sink);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_peak_read(const void *src, int64_t bytes, int32_t blocks, float *sink, st_stream stream) {
    st::clear_error();
    if (!src || !sink || bytes < 16 || bytes % 16 || blocks < 1 || (reinterpret_cast<uintptr_t>(src) & 15))
        return st::fail(ST_ERR_INVALID, "peak_read: need a 16-byte aligned buffer of a multiple of 16 bytes");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    hipLaunchKernelGGL(k_peak_read, dim3((unsigned)blocks), dim3(RT), 0, st::stream_of(stream),
                       reinterpret_cast<const float4 *>(src), bytes / 16, sink);
    ST_LAUNCH_CHECK();
    return ST_OK;
}

extern "C" st_status st_lane_selftest(uint32_t *out, st_stream stream) {
    st::clear_error();
    if (!out) return st::fail(ST_ERR_INVALID, "lane_selftest: NULL output");
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    hipLaunchKernelGGL(k_lane_selftest, dim3(1), dim3(64), 0, st::stream_of(stream), out);
    ST_LAUNCH_CHECK();
    return ST_OK;
}
