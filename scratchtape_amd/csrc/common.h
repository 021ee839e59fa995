// Internal helpers shared by the HIP translation units of libscratchtape_hip:
// error reporting through st_last_error(), HIP call checking, and the
// grow-only per-device scratch arena.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/scratchtape_hip.h"

namespace st {

// Sets the thread-local message returned by st_last_error() and returns `code`.
st_status fail(st_status code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread-local message (called on entry of each public function).
void clear_error();

// Device-resident scratch of at least `bytes` for work enqueued on `stream`.
// By default one grow-only arena per device and slot: growth allocates a new
// buffer (refused, with ST_ERR_INVALID, while `stream` is being captured into
// a graph) and keeps the superseded one until st_scratch_release(), since
// enqueued work or a captured graph may still use it.  Inside a ScratchScope
// the scope decides instead: a fixed buffer (sizes beyond it are refused), or
// private buffers that the scope frees when it ends (its owner synchronises
// the stream that used them first).  Returns nullptr and sets the error on
// failure.
enum ScratchSlot { SCRATCH_SPLITK = 0, SCRATCH_KNN = 1, SCRATCH_ROWS = 2, SCRATCH_SLOTS = 3 };
void *scratch(ScratchSlot slot, size_t bytes, hipStream_t stream);

// The status of this thread's last failed scratch() request (what a caller
// returns when scratch() gave nullptr).
st_status scratch_status();

// Redirects scratch() on this thread while alive (scopes nest).
class ScratchScope {
  public:
    ScratchScope(void *fixed, size_t bytes);  // every request served from [fixed, fixed + bytes)
    ScratchScope();                           // every request gets a private hipMalloc, freed at the end
    ~ScratchScope();
    ScratchScope(const ScratchScope &) = delete;
    ScratchScope &operator=(const ScratchScope &) = delete;

  private:
    friend void *scratch(ScratchSlot, size_t, hipStream_t);
    void *fixed_ = nullptr;
    size_t fixed_bytes_ = 0;
    ScratchScope *prev_;
    std::vector<void *> owned_;
};

// 1 when a gfx950 device is current; otherwise sets the error.
bool device_ok();

// The current device's compute-unit count (cached per device; 256 when the
// query fails).
int device_cus();

inline hipStream_t stream_of(st_stream s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace st

#define ST_HIP_CHECK(expr)                                                                  \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return ::st::fail(ST_ERR_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                              __FILE__, __LINE__);                                          \
    } while (0)

// Checks the launch that was just enqueued.
#define ST_LAUNCH_CHECK() ST_HIP_CHECK(hipGetLastError())
