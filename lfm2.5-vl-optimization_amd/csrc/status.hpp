// Host-side status plumbing shared by the entry points: per-thread error message, argument checks, launch checks,
// and the tuning knobs that force a kernel configuration.
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

// Tuning knobs: each forces one choice of a launch path (tile, split, kernel form) that is otherwise automatic.
// A knob holds up to four integers ("n" of them set; n == 0 = automatic). Initial values come from the environment
// variable of the same name, read once on first use; lfm2q_set_tuning changes them at run time. Every knob is one
// 64-bit atomic word, so a launch reads it with one load and never sees half of a concurrent update.
enum Knob {
    KNOB_GEMV_WPC,      // batch-1 persistent GEMV: wavefronts per CU
    KNOB_GEMV_PERSIST,  // batch-1 GEMV: 1 persistent, 0 one-shot kernel
    KNOB_GEMV_R,        // batch-1 one-shot GEMV: output rows per wavefront (1, 2, 4)
    KNOB_GEMV_VALU,     // batch-2 GEMV: 0 turns the VALU kernel off
    KNOB_GEMV_MFMA,     // batch 2..64 GEMV shape "KS,RT,NWK[,BT]"
    KNOB_GEMV_CHUNK,    // GEMV batch chunk (16 or 64 rows)
    KNOB_W4_WPC,        // batch-1 persistent INT4 GEMV: wavefronts per CU
    KNOB_W4_ONESHOT,    // batch-1 INT4 GEMV: 1 one-shot, 0 persistent kernel
    KNOB_W4_MFMA,       // INT4 batch 2..16 shape "KS,RT,NWK"
    KNOB_W4_B1_MFMA,    // INT4 batch 1 on the matrix-core kernel (1)
    KNOB_GEMM_BM,       // W8A8 / W8A16 tile rows
    KNOB_GEMM_BN,       // W8A8 / W8A16 tile columns
    KNOB_GEMM_KSPLIT,   // K split inside the workgroup (1, 2, 4)
    KNOB_GEMM_SWZ,      // XCD band traversal group (log2 of M-tiles per group)
    KNOB_GEMM_BIGP,     // 256 x 256 tiles: 0 = one workgroup per tile instead of the persistent kernel
    KNOB_GEMM_RING,     // 256 x 256 one-workgroup-per-tile ring shape (1282, 644, 645)
    KNOB_GEMM_STAGES,   // LDS ring depth (3, 6; 2 for the persistent kernels; 3 for the grouped kernel, default 4)
    KNOB_GEMM_SPLITK,   // per-token W8A8 with a workspace: K slices over workgroups (1 = none, 2..8)
    KNOB_CHAIN_WAIT_MS, // GEMV chain: bound of each dependency wait in milliseconds (default 20; 0: at once)
    KNOB_QUANT_WG,      // quant_rows / quant_groups: 1 a workgroup per row, 0 a wavefront per row
    KNOB_GEMM_FQ,       // gemm_i8_fq: 1 = the one-launch kernel (quantizing prologue); default 0, quant_rows + GEMM
    KNOB_GEMM_FQ_WAIT_US, // gemm_i8_fq prologue: microseconds before a waiting workgroup quantizes open chunks itself
    KNOB_GEMV_XS,       // batch-1 one-shot GEMV: 1 the activation row staged in LDS per workgroup, 0 per wavefront
    KNOB_GEMM_GSEQ,     // grouped 128 x 128 W8A8: 1 tile-sequential fold (three workgroups a CU), 0 pipelined fold
    KNOB_COUNT
};
struct KnobVal {
    int n;     // values set (0: automatic)
    int v[4];  // the values, v[i] = 0 for i >= n
};
KnobVal knob(Knob k);
// The knob's first value, or dflt when it is not set.
inline int knob_int(Knob k, int dflt) {
    const KnobVal kv = knob(k);
    return kv.n ? kv.v[0] : dflt;
}

}  // namespace lfm2q

#define LFM2Q_REQUIRE(cond, code, ...)                      \
    do {                                                    \
        if (!(cond)) return ::lfm2q::set_error(code, __VA_ARGS__); \
    } while (0)
