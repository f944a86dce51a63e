// Calibration for the grouped-64 W8A8 fold: can a SIMD run the fold's vector work (v_cvt_f32_i32 + v_fmac_f32 per
// accumulator) while its matrix core runs v_mfma_i32_32x32x32_i8, and what does that work cost on its own? Measurement
// equipment for bench.py (liblfm2q_calib.so), not part of the product interface.
//
// Each wavefront runs `iters` rounds of the grouped GEMM's per-stage work on a 64 x 64 wavefront block (four 32 x 32
// tiles): MFMA = 8 v_mfma_i32_32x32x32_i8 (two chained per tile), FOLD = 64 int32 -> fp32 conversions and 64 fp32
// FMAs on registers the MFMAs do not touch (plus 64 integer adds that keep the conversions' inputs changing), or both
// interleaved. Nothing depends across the two halves, so the "both" time against the two alone says how far the
// SIMD overlaps them. Results are folded into one store per lane so nothing can be removed.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <bool MF, bool FOLD>
__global__ __launch_bounds__(256) void fold_overlap_kernel(const int *__restrict__ in, int *__restrict__ out,
                                                            int iters) {
    const int lane = threadIdx.x & 63;
    v4i a = {in[lane], in[lane + 64], in[lane + 128], in[lane + 192]};
    const v4i b = a + 1;
    v16i acc[4] = {};
    float f[64];
    int src[64];
#pragma unroll
    for (int e = 0; e < 64; ++e) {
        f[e] = (float)(lane + e);
        src[e] = lane * e;
    }
    const float s = (float)in[lane + 256] * 1e-3f;
    for (int it = 0; it < iters; ++it) {
        if (MF) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, acc[t], 0, 0, 0);
            }
        }
        if (FOLD) {
#pragma unroll
            for (int e = 0; e < 64; ++e) f[e] = __builtin_fmaf((float)src[e], s, f[e]);
#pragma unroll
            for (int e = 0; e < 64; ++e) src[e] += 1;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    int r = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) r ^= acc[t][e];
    float fs = 0.f;
#pragma unroll
    for (int e = 0; e < 64; ++e) fs += f[e];
    out[blockIdx.x * 256 + threadIdx.x] = r ^ __float_as_int(fs);
}

}  // namespace

// mode 0: MFMA only, 1: fold only, 2: both. in: >= 512 int32 of device memory; out: blocks * 256 int32. Returns 0,
// -1 for bad arguments, -2 for a launch error.
extern "C" int lfm2q_calib_fold_overlap(int mode, const int *in, int *out, int blocks, int iters, hipStream_t stream) {
    if (!in || !out || blocks < 1 || iters < 1 || mode < 0 || mode > 2) return -1;
    if (mode == 0)
        fold_overlap_kernel<true, false><<<blocks, 256, 0, stream>>>(in, out, iters);
    else if (mode == 1)
        fold_overlap_kernel<false, true><<<blocks, 256, 0, stream>>>(in, out, iters);
    else
        fold_overlap_kernel<true, true><<<blocks, 256, 0, stream>>>(in, out, iters);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
