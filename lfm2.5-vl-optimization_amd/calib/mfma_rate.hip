// Calibration for the W8A8 roofline: the int8 matrix-core rate the chip sustains when every SIMD does nothing but
// v_mfma_i32_32x32x32_i8, and the shader clock it runs at meanwhile. A separate library (liblfm2q_calib.so): it is
// measurement equipment for bench.py, not part of the product interface.
//
// Each wavefront loads 4 A and 4 B fragments (16 bytes per lane each) once from `src`, then runs `iters` rounds of 8
// independent MFMAs (8 accumulator chains, enough to issue back to back), and writes a per-lane checksum of its
// accumulators to `out` so the work cannot be removed. The operand bytes decide the switching activity, and with it
// the power draw and the clock: bench.py runs random bytes (what a GEMM sees) and zeros.
//
// Lane 0 of wavefront 0 of workgroup 0 also records s_memrealtime (a constant 100 MHz) and s_memtime (the shader
// clock) before and after its loop: their ratio is the clock during the run.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int THREADS = 256;  // 4 wavefronts per workgroup
constexpr int FRAG_PER_WAVE = 8;

__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma_i8_rate_kernel(const v4i *__restrict__ src, int32_t *__restrict__ out,
                                                               uint64_t *__restrict__ clocks, int iters) {
    const int lane = threadIdx.x & 63;
    const int gw = (int)((blockIdx.x * THREADS + threadIdx.x) >> 6);  // global wavefront index
    v4i a[4], b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        a[q] = src[(size_t)(gw * FRAG_PER_WAVE + q) * 64 + lane];
        b[q] = src[(size_t)(gw * FRAG_PER_WAVE + 4 + q) * 64 + lane];
    }
    v16i acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[c][e] = 0;
    const bool timer = blockIdx.x == 0 && threadIdx.x == 0;
    uint64_t r0 = 0, c0 = 0;
    if (timer) {
        r0 = __builtin_amdgcn_s_memrealtime();
        c0 = __builtin_amdgcn_s_memtime();
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[c & 3], b[c >> 1], acc[c], 0, 0, 0);
    }
    if (timer) {
        const uint64_t r1 = __builtin_amdgcn_s_memrealtime(), c1 = __builtin_amdgcn_s_memtime();
        clocks[0] = r1 - r0;
        clocks[1] = c1 - c0;
    }
    int32_t s = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[c][e];
    out[(size_t)gw * 64 + lane] = s;
}

}  // namespace

// blocks workgroups of 4 wavefronts (8 per CU for two wavefronts per SIMD: blocks = 2 x the CU count).
// src: at least blocks x 4 x 8 KiB of operand bytes; out: blocks x 256 int32; clocks: 2 uint64 (real-time ticks
// at 100 MHz, shader clock ticks). Returns 0, or -1 for a size that does not fit the buffers, -2 for a launch error.
// The work is blocks x 4 x iters x 8 MFMAs of 2 x 32 x 32 x 32 = 65536 int8 ops each.
extern "C" int lfm2q_calib_mfma_i8(const void *src, size_t src_bytes, int32_t *out, size_t out_bytes,
                                   uint64_t *clocks, int blocks, int iters, hipStream_t stream) {
    if (!src || !out || !clocks || blocks < 1 || iters < 1) return -1;
    const size_t waves = (size_t)blocks * (THREADS / 64);
    if (src_bytes < waves * FRAG_PER_WAVE * 64 * 16 || out_bytes < waves * 64 * 4 || ((uintptr_t)src & 15)) return -1;
    mfma_i8_rate_kernel<<<blocks, THREADS, 0, stream>>>(static_cast<const v4i *>(src), out, clocks, iters);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
