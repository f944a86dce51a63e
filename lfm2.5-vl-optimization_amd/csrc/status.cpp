#include "status.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

namespace lfm2q {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

int launch_status(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(LFM2Q_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return LFM2Q_OK;
}

}  // namespace lfm2q

extern "C" const char *lfm2q_last_error(void) { return lfm2q::g_err; }
extern "C" const char *lfm2q_version(void) { return "lfm2q 0.1.0 (gfx950)"; }
