// Symmetric INT8 quantization of bf16 values, shared by the standalone quantizers, the fused producers and the
// INT8-output GEMM epilogue, so every path that quantizes the same bf16 values produces the same bytes.
#pragma once

#include "common.hpp"

namespace lfm2q {

// q = rint(x / s) with round-half-even (the reference's integer clamp to [-127, 127] never binds: |x| <= amax keeps
// |x / s| < 127.5). x / s is evaluated as t = x * fl(1 / s): two roundings put t within 127.5 * 2^-23 < 2^-16 of the
// real quotient, and the correctly rounded quotient fl(x / s) is within half an ulp (<= 2^-17) of it, so unless t
// lies within 2^-15 of a half-integer, rint(t) and rint(fl(x / s)) are the same integer. Near a half-integer the
// IEEE quotient itself is computed; the test runs per 8 values and the division only when one of them needs it.
// The test reuses the rounding: with d = t - rint(t) (exact, Sterbenz: |d| <= 0.5 <= |rint(t)| / 2 unless rint(t) =
// 0, where d = t), |d| = 0.5 - |f - 0.5| for the fraction f of t, so |d| > 0.5 - 2^-15 exactly when t is within 2^-15
// of a half-integer (ties give |d| = 0.5).
constexpr float NEAR_HALF = 0.5f - 0.000030517578125f;  // 0.5 - 2^-15, exact in fp32

// 8 bf16 (one 16-byte vector) -> 8 int8 packed in two dwords
__device__ __forceinline__ void quant8(v4i xv, float s, float r, int &lo, int &hi) {
    float v[8], t[8], rt[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[2 * j] = bf2f_lo((uint32_t)xv[j]);
        v[2 * j + 1] = bf2f_hi((uint32_t)xv[j]);
    }
    bool any = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        t[e] = v[e] * r;
        rt[e] = rintf(t[e]);
        any |= fabsf(t[e] - rt[e]) > NEAR_HALF;
    }
    if (__builtin_expect(any, 0)) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (fabsf(t[e] - rt[e]) > NEAR_HALF) rt[e] = rintf(v[e] / s);
    }
    // the low byte of each integer, four per dword (v_perm: selector 0x00-0x03 picks a byte of the second operand,
    // 0x04-0x07 of the first, 0x0c gives 0)
    uint32_t q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = (uint32_t)(int)rt[e];
    lo = (int)(__builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u) | __builtin_amdgcn_perm(q[3], q[2], 0x04000c0cu));
    hi = (int)(__builtin_amdgcn_perm(q[5], q[4], 0x0c0c0400u) | __builtin_amdgcn_perm(q[7], q[6], 0x04000c0cu));
}

__device__ __forceinline__ float absmax8(v4i xv, float m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf2f_lo((uint32_t)xv[j])), fabsf(bf2f_hi((uint32_t)xv[j]))));
    return m;
}

__device__ __forceinline__ float scale_of(float amax) { return fmaxf(amax, 1e-8f) / 127.f; }

// s[r] = quant_rows' scale of row r of x (bf16 [rows, K], K % 8 == 0), on `st` (quant.hip)
int launch_row_scales(const uint16_t *x, float *s, int rows, int K, hipStream_t st);

}  // namespace lfm2q
