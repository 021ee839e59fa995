// Library runtime: error reporting, device check, scratch arena, version.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"

namespace st {

static thread_local std::string g_error;

st_status fail(st_status code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

void clear_error() { g_error.clear(); }

namespace {
struct Arena {
    void *ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_arena_mu;
std::vector<Arena> g_arenas;  // [device * SCRATCH_SLOTS + slot]
}  // namespace

void *scratch(ScratchSlot slot, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        fail(ST_ERR_HIP, "hipGetDevice failed");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_arena_mu);
    size_t i = (size_t)dev * SCRATCH_SLOTS + slot;
    if (g_arenas.size() <= i) g_arenas.resize(i + 1);
    Arena &a = g_arenas[i];
    if (a.bytes >= bytes && a.ptr) return a.ptr;
    size_t grow = bytes + bytes / 4;  // headroom: sizes vary a little per call
    grow = (grow + 255) & ~(size_t)255;
    if (a.ptr) {
        (void)hipFree(a.ptr);  // synchronises the device: no enqueued work still reads it
        a.ptr = nullptr;
        a.bytes = 0;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, grow);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(ST_ERR_OOM, "scratch arena could not grow to %zu bytes: %s", grow, hipGetErrorString(e));
        return nullptr;
    }
    a.ptr = p;
    a.bytes = grow;
    return p;
}

bool device_ok() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        fail(ST_ERR_NO_DEVICE, "no HIP device visible");
        return false;
    }
    static thread_local int checked_dev = -1;
    if (checked_dev == dev) return true;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        fail(ST_ERR_NO_DEVICE, "hipGetDeviceProperties failed");
        return false;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        fail(ST_ERR_NO_DEVICE, "libscratchtape_hip is built for gfx950 only; device %d is %s", dev,
             prop.gcnArchName);
        return false;
    }
    checked_dev = dev;
    return true;
}

}  // namespace st

extern "C" const char *st_last_error(void) { return st::g_error.c_str(); }

extern "C" st_status st_sync(st_stream stream) {
    st::clear_error();
    ST_HIP_CHECK(hipStreamSynchronize(st::stream_of(stream)));
    return ST_OK;
}

extern "C" const char *st_version(void) { return "scratchtape_hip 0.1.0 (gfx950)"; }
