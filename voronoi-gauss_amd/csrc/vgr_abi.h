// Host-side helpers of the C ABI: thread-local error message and launch-status checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/vgr.h"

namespace vgr {

// Records the message (printf format) for vgr_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// VGR_OK if the last launch on this thread succeeded, else VGR_ERR_LAUNCH with the runtime's message.
int launch_status(const char* kernel);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Grid size for n work items of `per_block` items each; 0 when n == 0.
inline unsigned grid_for(int64_t n, int per_block) { return static_cast<unsigned>((n + per_block - 1) / per_block); }

}  // namespace vgr

#define VGR_REQUIRE(cond, ...)                                      \
    do {                                                            \
        if (!(cond)) return ::vgr::fail(VGR_ERR_INVALID, __VA_ARGS__); \
    } while (0)
