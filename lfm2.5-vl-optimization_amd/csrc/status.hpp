// Host-side status plumbing shared by the entry points: per-thread error message, argument checks, launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lfm2q.h"

namespace lfm2q {

int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Launch status: LFM2Q_OK, or LFM2Q_ERR_LAUNCH with the HIP error string recorded.
int launch_status(const char *what);

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace lfm2q

#define LFM2Q_REQUIRE(cond, code, ...)                      \
    do {                                                    \
        if (!(cond)) return ::lfm2q::set_error(code, __VA_ARGS__); \
    } while (0)
