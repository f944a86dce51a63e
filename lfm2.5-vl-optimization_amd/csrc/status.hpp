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

// Compute units of the current device (queried once per device, then cached; 256 on MI355X).
int device_cus();

// Integer tuning knob from the environment (read once per name by the caller), or `dflt` when unset.
int env_int(const char *name, int dflt);

}  // namespace lfm2q

#define LFM2Q_REQUIRE(cond, code, ...)                      \
    do {                                                    \
        if (!(cond)) return ::lfm2q::set_error(code, __VA_ARGS__); \
    } while (0)
