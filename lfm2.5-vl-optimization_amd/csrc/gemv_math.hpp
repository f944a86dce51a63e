// Per-row arithmetic of the batch-1 decode GEMVs, shared by the single-GEMV kernels (gemv.hip) and the GEMV chain
// (chain.hip) so that both compute every output row with the same instructions in the same order, and so give the
// same bits: int8 / bf16 weight chunks against bf16 activation pairs on v_dot2_f32_bf16, and the epilogues.
#pragma once
#include "common.hpp"

namespace lfm2q {

enum Epi { EPI_NONE = 0, EPI_SWIGLU = 1, EPI_RESIDUAL = 2 };

// ------------------------------------------------------------------------------------------------ chunk math
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2bf as_bf16x2(uint32_t v) { return __builtin_bit_cast(v2bf, v); }
// the upper halves of two fp32 values as one bf16 pair (lo in bits 0-15): v_perm_b32 takes bytes 2, 3 of `lo`
// (selectors 2, 3) and bytes 2, 3 of `hi` (selectors 6, 7); exact when both values are bf16-representable
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
// acc + sum of one 16-byte weight chunk times its activations, the activations given as bf16 pairs (the chunk's
// PER values, packed as loaded). int8 weights are converted exactly to bf16 pairs; v_dot2_f32_bf16 multiplies and
// adds a pair per instruction with fp32 accumulation, so the activations are never unpacked.
template <typename WT>
struct PairDot;
template <>
struct PairDot<int8_t> {
    static constexpr int PER = 16, XL = 2;  // 16 weights, activations in two 16-byte vectors
    __device__ static float dot(v4i c, const v4i *xq, float acc) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = c[j];
            const uint32_t p0 = pack_hi16((float)(int8_t)d, (float)(int8_t)(d >> 8));
            const uint32_t p1 = pack_hi16((float)(int8_t)(d >> 16), (float)(d >> 24));
            a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(p0), as_bf16x2((uint32_t)xq[j >> 1][2 * (j & 1)]), a, false);
            a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(p1), as_bf16x2((uint32_t)xq[j >> 1][2 * (j & 1) + 1]), a,
                                                false);
        }
        return acc + a;
    }
};
template <>
struct PairDot<uint16_t> {
    static constexpr int PER = 8, XL = 1;
    __device__ static float dot(v4i c, const v4i *xq, float acc) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2((uint32_t)c[j]), as_bf16x2((uint32_t)xq[0][j]), a, false);
        return acc + a;
    }
};

// The value stored for one output row from its fp32 sum(s): EPI_NONE y = bf16(r s); EPI_RESIDUAL y = bf16(h +
// bf16(r s)) (the reference's residual rounding, kernels/lfm2_decode.cu:108-113); EPI_SWIGLU y = bf16(bf16(silu(g))
// u) with g = bf16(r s), u = bf16(ru su) (kernels/lfm2_decode.cu:786-790 and :954-963). scale == false: s = su = 1.
template <int EPI>
__device__ __forceinline__ uint16_t gemv_epilogue(float r, float sg, float ru, float su, uint32_t h, bool scaled) {
    if (EPI == EPI_NONE) return (uint16_t)f2bf(scaled ? r * sg : r);
    if (EPI == EPI_RESIDUAL) return (uint16_t)f2bf(bf2f(h) + rbf(scaled ? r * sg : r));
    const float g = rbf(scaled ? r * sg : r), u = rbf(scaled ? ru * su : ru);
    return (uint16_t)f2bf(rbf(silu_f32(g)) * u);
}

}  // namespace lfm2q
