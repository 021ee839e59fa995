// st_matmul_grouped_noalloc: st_matmul_grouped for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  Its split-k partials live in `scratch`, a
// fixed device array of this file, instead of the library's grow-only arena;
// the kernels are those of st_matmul_grouped and take the array's device
// address as they take an arena buffer.
//
// The array is per device (each GPU the library runs on holds its own copy
// until the process ends) and shared by every call on that device: calls that
// overlap on one device race on it.  Nothing in it needs clearing between
// calls: each split slice writes all of its partials before the sums read
// them.
#include <mutex>

#include "common.h"

static __device__ __align__(256) unsigned char scratch[ST_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES];  // device address of `scratch` per device, 0 until looked up

// The device address of the current device's copy of `scratch`.  In host code
// the array's name is only a host-side stand-in, so the address is looked up
// once per device, with that device current, and kept.
st_status scratch_ptr(void **out) {
    int dev = 0;
    ST_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return st::fail(ST_ERR_NO_DEVICE, "device %d: more devices than supported", dev);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return st::fail(ST_ERR_HIP, "hipGetSymbolAddress of the fixed scratch failed: %s", hipGetErrorString(e));
        }
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return ST_OK;
}

}  // namespace

extern "C" st_status st_matmul_grouped_noalloc(const st_gemm *gemms, int64_t count, st_stream stream) {
    st::clear_error();
    if (count < 0 || (count > 0 && !gemms)) return st::fail(ST_ERR_INVALID, "grouped GEMM: bad count or NULL array");
    if (count == 0) return ST_OK;
    if (!st::device_ok()) return ST_ERR_NO_DEVICE;
    void *p = nullptr;
    const st_status s = scratch_ptr(&p);
    if (s != ST_OK) return s;
    st::ScratchScope fixed(p, ST_NOALLOC_SCRATCH_BYTES);
    return st_matmul_grouped(gemms, count, stream);
}
