// Host-side helpers for the C ABI: the thread-local last error and the HIP
// launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "zest_hip.h"

namespace zest {

// Sets the calling thread's last error and returns `status`.
int fail(int status, const char * fmt, ...) __attribute__((format(printf, 2, 3)));

inline hipStream_t as_stream(void * s) { return reinterpret_cast<hipStream_t>(s); }

// Non-zero when the last launch failed (the error is recorded).
int check_launch(const char * what);

// Looks up, with `dev` current, the device address of the no-alloc entry
// point's static workspace on that device (once per device; zest_init calls it).
int scratch_setup(int dev);

// Devices the per-device tables hold.
#define ZEST_MAX_DEVICES 64

} // namespace zest

#define ZEST_REQUIRE(cond, ...)                               \
    do {                                                      \
        if (!(cond)) return zest::fail(ZEST_E_ARG, __VA_ARGS__); \
    } while (0)
