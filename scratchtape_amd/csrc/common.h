// Internal helpers shared by the HIP translation units of libscratchtape_hip:
// error reporting through st_last_error(), HIP call checking, and the
// grow-only per-device scratch arena.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/scratchtape_hip.h"

namespace st {

// Sets the thread-local message returned by st_last_error() and returns `code`.
st_status fail(st_status code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread-local message (called on entry of each public function).
void clear_error();

// Device-resident scratch of at least `bytes`, grown on demand (hipMalloc of
// the new size; the old buffer is freed, which synchronises the device).
// Never shrinks.  One arena per device and slot.  Returns nullptr and sets the
// error on failure.
enum ScratchSlot { SCRATCH_SPLITK = 0, SCRATCH_KNN = 1, SCRATCH_ROWS = 2, SCRATCH_SLOTS = 3 };
void *scratch(ScratchSlot slot, size_t bytes);

// 1 when a gfx950 device is current; otherwise sets the error.
bool device_ok();

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
