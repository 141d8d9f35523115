// Error reporting shared by every C-ABI entry point of libh3vae_hip.so.
//
// Entry points return H3V_OK (0) or a nonzero code; the message of the last
// failure on the calling thread is available through h3v_last_error().
// Argument checks run on the host before any launch, so a rejected call has
// queued no GPU work.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/h3vae_hip.h"

namespace h3v {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError after a launch and converts it into an error code.
int launch_status(const char* what);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace h3v

#define H3V_REQUIRE(cond, ...)                                   \
    do {                                                         \
        if (!(cond)) return ::h3v::fail(H3V_EINVAL, __VA_ARGS__); \
    } while (0)
