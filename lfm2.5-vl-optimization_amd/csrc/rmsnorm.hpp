// RMSNorm arithmetic shared by the add_rmsnorm_q producer (quant.hip) and the batch-1 GEMVs that normalize their
// input row themselves (gemv.hip), so that both produce the same bits: x = bf16(w * bf16(h * rs)),
// rs = 1 / sqrt(sum(h^2) / H + eps), the sum taken per lane over the 8-value vectors c 64 + lane (c = 0, 1, ...) in
// element order, each product rounded before it is added, then across the wavefront by wave_sum. Contraction is off
// so that every rounding is the one written (transformers' Lfm2RMSNorm rounding points, as add_rmsnorm_q has them).
#pragma once
#include "common.hpp"

namespace lfm2q {

// ss + the squares of the 8 bf16 values of one vector, in element order
__device__ __forceinline__ float sumsq8(v4i hv, float ss) {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = bf2f_lo((uint32_t)hv[j]), b = bf2f_hi((uint32_t)hv[j]);
        ss += a * a;
        ss += b * b;
    }
    return ss;
}

// rs from the wavefront's total sum of squares over a row of H values
__device__ __forceinline__ float rms_scale(float ss, int H, float eps) {
#pragma clang fp contract(off)
    return 1.f / sqrtf(ss / (float)H + eps);
}

// one dword of x (two bf16) from the matching dwords of the norm weight and of h
__device__ __forceinline__ uint32_t rms_apply2(uint32_t w, uint32_t h, float rs) {
#pragma clang fp contract(off)
    return pack_bf16x2(bf2f_lo(w) * rbf(bf2f_lo(h) * rs), bf2f_hi(w) * rbf(bf2f_hi(h) * rs));
}

}  // namespace lfm2q
