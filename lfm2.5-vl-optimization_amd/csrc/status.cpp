#include "status.hpp"

#include <atomic>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

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
    static std::atomic<int> cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

int launch_status(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(LFM2Q_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return LFM2Q_OK;
}

// ------------------------------------------------------------------------------------------------ tuning knobs
namespace {

const char *const kKnobNames[KNOB_COUNT] = {
    "LFM2Q_GEMV_WPC",  "LFM2Q_GEMV_PERSIST", "LFM2Q_GEMV_R",   "LFM2Q_GEMV_VALU",    "LFM2Q_GEMV_MFMA",
    "LFM2Q_GEMV_CHUNK", "LFM2Q_W4_WPC",      "LFM2Q_W4_ONESHOT", "LFM2Q_W4_MFMA",    "LFM2Q_W4_B1_MFMA",
    "LFM2Q_GEMM_BM",   "LFM2Q_GEMM_BN",      "LFM2Q_GEMM_KSPLIT", "LFM2Q_GEMM_SWZ",   "LFM2Q_GEMM_BIGP",
    "LFM2Q_GEMM_RING", "LFM2Q_GEMM_STAGES", "LFM2Q_GEMM_SPLITK", "LFM2Q_CHAIN_WAIT_MS",
    "LFM2Q_QUANT_WG", "LFM2Q_GEMM_FQ", "LFM2Q_GEMM_FQ_WAIT_US", "LFM2Q_GEMV_XS", "LFM2Q_GEMM_GSEQ",
};

// A knob word: bits 0-3 the count n, value i (signed, |v| < 16384) in bits 4 + 15 i .. 18 + 15 i.
std::atomic<uint64_t> g_knobs[KNOB_COUNT];
std::once_flag g_knobs_env;

constexpr int kKnobMax = 16383;

// "a,b,c" -> packed word; false if it is not 1..4 comma-separated integers within range
bool parse_knob(const char *s, uint64_t *out) {
    uint64_t w = 0;
    int n = 0;
    const char *p = s;
    while (*p) {
        if (n == 4) return false;
        char *end = nullptr;
        const long v = strtol(p, &end, 10);
        if (end == p || v < -kKnobMax || v > kKnobMax) return false;
        w |= (uint64_t)((uint32_t)v & 0x7fffu) << (4 + 15 * n);
        ++n;
        p = end;
        if (*p == ',') {
            ++p;
            if (!*p) return false;
        } else if (*p) {
            return false;
        }
    }
    *out = n ? (w | (uint64_t)n) : 0;
    return true;
}

void read_env_knobs() {
    for (int k = 0; k < KNOB_COUNT; ++k) {
        const char *e = getenv(kKnobNames[k]);
        uint64_t w = 0;
        if (e && *e && parse_knob(e, &w)) g_knobs[k].store(w, std::memory_order_relaxed);
    }
}

}  // namespace

KnobVal knob(Knob k) {
    std::call_once(g_knobs_env, read_env_knobs);
    const uint64_t w = g_knobs[k].load(std::memory_order_relaxed);
    KnobVal r{(int)(w & 15u), {0, 0, 0, 0}};
    for (int i = 0; i < r.n; ++i) {
        const int v = (int)((w >> (4 + 15 * i)) & 0x7fffu);
        r.v[i] = v >= 0x4000 ? v - 0x8000 : v;
    }
    return r;
}

}  // namespace lfm2q

using namespace lfm2q;

extern "C" const char *lfm2q_last_error(void) { return g_err; }
extern "C" const char *lfm2q_version(void) { return "lfm2q 0.2.0 (gfx950)"; }

extern "C" int lfm2q_set_tuning(const char *name, const char *value) {
    LFM2Q_REQUIRE(name, LFM2Q_ERR_ARG, "set_tuning: null knob name");
    std::call_once(g_knobs_env, read_env_knobs);
    for (int k = 0; k < KNOB_COUNT; ++k) {
        if (strcmp(name, kKnobNames[k]) != 0) continue;
        uint64_t w = 0;
        if (value && *value && !parse_knob(value, &w))
            return set_error(LFM2Q_ERR_ARG, "set_tuning: %s: expected 1 to 4 comma-separated integers, got '%s'",
                             name, value);
        g_knobs[k].store(w, std::memory_order_relaxed);
        return LFM2Q_OK;
    }
    return set_error(LFM2Q_ERR_ARG, "set_tuning: unknown knob '%s'", name);
}

extern "C" int lfm2q_get_tuning(const char *name, int *values, int *count) {
    LFM2Q_REQUIRE(name && values && count, LFM2Q_ERR_ARG, "get_tuning: null pointer");
    for (int k = 0; k < KNOB_COUNT; ++k) {
        if (strcmp(name, kKnobNames[k]) != 0) continue;
        const KnobVal kv = knob((Knob)k);
        *count = kv.n;
        for (int i = 0; i < 4; ++i) values[i] = kv.v[i];
        return LFM2Q_OK;
    }
    return set_error(LFM2Q_ERR_ARG, "get_tuning: unknown knob '%s'", name);
}
