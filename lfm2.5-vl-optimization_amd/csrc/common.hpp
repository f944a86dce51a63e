// Shared device helpers for the gfx950 kernels of liblfm2q: bf16 <-> fp32 with explicit rounding, wave64
// reductions, non-temporal 16-byte loads and the MFMA operand vector types.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lfm2q {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// bf16 is carried as its raw 16-bit pattern everywhere (uint16_t); conversions are done by hand so that the
// rounding mode is explicit: fp32 -> bf16 is round-to-nearest-even, NaN stays a quiet NaN.
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf2f_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf2f_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }  // round to bf16 and back

// Sum over the 64 lanes of a wave; every lane receives the total. The butterfly order is fixed, so the result is
// a deterministic function of the 64 inputs (kernels that must agree bit for bit share this routine).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// 16-byte streaming load that does not keep the line in the caches (weights are read exactly once per call).
__device__ __forceinline__ v4i ld_nt16(const void *p) { return __builtin_nontemporal_load((const v4i *)p); }
// 16-byte cached load (activations: small and shared by every wave).
__device__ __forceinline__ v4i ld16(const void *p) { return *(const v4i *)p; }

// SiLU exactly as the decode path rounds it: silu(g) = g / (1 + exp(-g)) in fp32.
__device__ __forceinline__ float silu_f32(float g) { return g / (1.f + expf(-g)); }

// GELU, tanh approximation, in fp32: 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))).
__device__ __forceinline__ float gelu_tanh_f32(float v) {
    return 0.5f * v * (1.f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

}  // namespace lfm2q
