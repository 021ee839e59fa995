// Library runtime: error reporting, device check, scratch arena, version.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"
#include "gemm_dma.h"

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
std::vector<Arena> g_arenas;      // [device * SCRATCH_SLOTS + slot]
std::vector<void *> g_retired;    // superseded arena buffers, kept until st_scratch_release
thread_local ScratchScope *g_scope = nullptr;
thread_local st_status g_scratch_status = ST_OK;
}  // namespace

st_status scratch_status() { return g_scratch_status; }

ScratchScope::ScratchScope(void *fixed, size_t bytes) : fixed_(fixed), fixed_bytes_(bytes), prev_(g_scope) {
    g_scope = this;
}

ScratchScope::ScratchScope() : prev_(g_scope) { g_scope = this; }

// The owner of a private scope has synchronised the stream its work went to
// before the scope ends (st_ndarray_matmul does), so the buffers are idle:
// no device-wide synchronisation, which would also wait for other threads'
// streams.
ScratchScope::~ScratchScope() {
    g_scope = prev_;
    for (void *p : owned_) (void)hipFree(p);
}

void *scratch(ScratchSlot slot, size_t bytes, hipStream_t stream) {
    if (bytes == 0) bytes = 256;
    if (ScratchScope *sc = g_scope) {
        if (sc->fixed_) {
            // One buffer for the whole call: the slots' uses in one call are
            // never in flight together (each is used by one entry point).
            if (bytes > sc->fixed_bytes_) {
                g_scratch_status = ST_ERR_INVALID;
                fail(ST_ERR_INVALID, "call needs %zu bytes of scratch; the fixed scratch holds %zu", bytes,
                     sc->fixed_bytes_);
                return nullptr;
            }
            return sc->fixed_;
        }
        void *p = nullptr;
        const hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            g_scratch_status = ST_ERR_OOM;
            fail(ST_ERR_OOM, "private scratch of %zu bytes could not be allocated: %s", bytes, hipGetErrorString(e));
            return nullptr;
        }
        sc->owned_.push_back(p);
        return p;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        g_scratch_status = ST_ERR_HIP;
        fail(ST_ERR_HIP, "hipGetDevice failed");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_arena_mu);
    size_t i = (size_t)dev * SCRATCH_SLOTS + slot;
    if (g_arenas.size() <= i) g_arenas.resize(i + 1);
    Arena &a = g_arenas[i];
    if (a.bytes >= bytes && a.ptr) return a.ptr;
    // Growing allocates device memory, which a stream under graph capture
    // must not do: the graph would hold a buffer the next growth replaces.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) {
        (void)hipGetLastError();
        cap = hipStreamCaptureStatusNone;
    }
    if (cap != hipStreamCaptureStatusNone) {
        g_scratch_status = ST_ERR_INVALID;
        fail(ST_ERR_INVALID,
             "scratch arena would have to grow to %zu bytes while the stream is being captured into a graph: run "
             "the same call once before capturing it",
             bytes);
        return nullptr;
    }
    size_t grow = bytes + bytes / 4;  // headroom: sizes vary a little per call
    grow = (grow + 255) & ~(size_t)255;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, grow);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        g_scratch_status = ST_ERR_OOM;
        fail(ST_ERR_OOM, "scratch arena could not grow to %zu bytes: %s", grow, hipGetErrorString(e));
        return nullptr;
    }
    // The old buffer may still be read by enqueued work or by a captured graph
    // that will be replayed: it is kept until st_scratch_release.
    if (a.ptr) g_retired.push_back(a.ptr);
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

int device_cus() {
    constexpr int MAX_DEVICES = 64;
    static std::atomic<int> cached[MAX_DEVICES];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return 256;
    }
    if (dev >= 0 && dev < MAX_DEVICES) {
        const int c = cached[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
        (void)hipGetLastError();
        return 256;
    }
    if (dev >= 0 && dev < MAX_DEVICES) cached[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

}  // namespace st

extern "C" const char *st_last_error(void) { return st::g_error.c_str(); }

extern "C" st_status st_sync(st_stream stream) {
    st::clear_error();
    ST_HIP_CHECK(hipStreamSynchronize(st::stream_of(stream)));
    return st::check_group_waits();
}

extern "C" st_status st_scratch_release(void) {
    st::clear_error();
    std::lock_guard<std::mutex> lock(st::g_arena_mu);
    int cur = 0;
    ST_HIP_CHECK(hipGetDevice(&cur));
    int ndev = 0;
    ST_HIP_CHECK(hipGetDeviceCount(&ndev));
    for (int d = 0; d < ndev; d++) {
        bool any = false;
        for (int slot = 0; slot < st::SCRATCH_SLOTS; slot++) {
            const size_t i = (size_t)d * st::SCRATCH_SLOTS + slot;
            any = any || (i < st::g_arenas.size() && st::g_arenas[i].ptr);
        }
        if (!any && (d != cur || st::g_retired.empty())) continue;
        ST_HIP_CHECK(hipSetDevice(d));
        ST_HIP_CHECK(hipDeviceSynchronize());
    }
    ST_HIP_CHECK(hipSetDevice(cur));
    // hipFree of a buffer of another device is fine from any current device.
    for (void *p : st::g_retired) (void)hipFree(p);
    st::g_retired.clear();
    for (st::Arena &a : st::g_arenas) {
        if (a.ptr) (void)hipFree(a.ptr);
        a = st::Arena();
    }
    return ST_OK;
}

extern "C" const char *st_version(void) { return "scratchtape_hip 0.1.0 (gfx950)"; }
