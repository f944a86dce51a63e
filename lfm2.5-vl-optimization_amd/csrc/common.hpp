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

// bf16 is carried as its raw 16-bit pattern everywhere (uint16_t). fp32 -> bf16 is gfx950's v_cvt_pk_bf16_f32
// (one instruction per pair of values): round to nearest even, and a NaN becomes the quiet NaN with its sign and
// upper payload, i.e. for every fp32 pattern u the bits of the explicit formula
//   NaN: (u >> 16) | 0x40,   otherwise: (u + 0x7fff + ((u >> 16) & 1)) >> 16
// (checked on the device against that formula over 2^20 patterns spanning every exponent, with the NaN, denormal,
// tie and overflow cases), which is how the CPU oracle rounds.
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf2f_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf2f_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }  // round to bf16 and back
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {  // lo in bits 0-15, hi in bits 16-31
    const v2bf r = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, r);
}

// DPP lane permutations within a 16-lane row (no LDS traffic, unlike ds_bpermute).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int DPP_XOR1 = 0xb1;         // quad_perm [1, 0, 3, 2]
constexpr int DPP_XOR2 = 0x4e;         // quad_perm [2, 3, 0, 1]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <- lane 7 - i within each 8 lanes
constexpr int DPP_MIRROR = 0x140;       // lane i <- lane 15 - i within each 16 lanes

__device__ __forceinline__ float lane_read(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the 64 lanes of a wave; every lane receives the total. The order is fixed (row sums by DPP, then the
// four row sums added as (r0 + r1) + (r2 + r3)), so the result is a deterministic function of the 64 inputs:
// kernels that must agree bit for bit share this routine.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<DPP_XOR1>(v);
    v += dpp<DPP_XOR2>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    v += dpp<DPP_MIRROR>(v);
    return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<DPP_XOR1>(v));
    v = fmaxf(v, dpp<DPP_XOR2>(v));
    v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp<DPP_MIRROR>(v));
    return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}

// Sums of V values (V = 1, 2, 4, 8) over the 64 lanes of a wavefront in one transposed reduction: lane bits 5, 4
// and 3 are folded first -- while several values remain, each fold pairs two of them, so that half the lanes add
// the partner's copy of one value and the other half of the other (permlane32 / permlane16 swaps, then a DPP row
// rotation by 8) -- then bits 0, 1 and 2 by DPP within 8 lanes. Value v ends in lanes v 64 / V .. v 64 / V + 64 / V
// - 1. The lane pairing is the same for every V and slot, so a value's sum does not depend on how many values
// share the call (8 values cost about as much as 2 separate wave sums).
constexpr int DPP_ROR8 = 0x128;  // lane i <- lane i ^ 8 within each 16 lanes (row rotation by 8)
template <int V>
__device__ __forceinline__ float fold_sum(const float (&v)[V]) {
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "fold_sum: V in {1, 2, 4, 8}");
    constexpr int V1 = V >= 2 ? V / 2 : 1, V2 = V1 >= 2 ? V1 / 2 : 1;
    float b[V1], c[V2];
#pragma unroll
    for (int i = 0; i < V1; ++i) {  // bit 5: lanes 0-31 keep value i, lanes 32-63 value i + V1
        const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[V >= 2 ? i + V1 : i]),
                                                        false, false);
        b[i] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    }
#pragma unroll
    for (int i = 0; i < V2; ++i) {  // bit 4: even 16-lane rows keep b[i], odd rows b[i + V2]
        const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(b[i]), __float_as_uint(b[V1 >= 2 ? i + V2 : i]),
                                                        false, false);
        c[i] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    }
    float d;  // bit 3
    if constexpr (V2 >= 2) {
        const bool hi = (threadIdx.x & 8) != 0;
        d = (hi ? c[1] : c[0]) + dpp<DPP_ROR8>(hi ? c[0] : c[1]);
    } else {
        d = c[0] + dpp<DPP_ROR8>(c[0]);
    }
    d += dpp<DPP_XOR1>(d);
    d += dpp<DPP_XOR2>(d);
    d += dpp<DPP_HALF_MIRROR>(d);
    return d;
}

// 16-byte streaming load that does not keep the line in the caches (weights are read exactly once per call).
__device__ __forceinline__ v4i ld_nt16(const void *p) { return __builtin_nontemporal_load((const v4i *)p); }
// 16-byte cached load (activations: small and shared by every wave).
__device__ __forceinline__ v4i ld16(const void *p) { return *(const v4i *)p; }

// Buffer resources (gfx9 descriptor word 3 = 0x00020000): a wavefront-uniform base and byte range held in four
// SGPRs. Loads through them take a per-lane byte offset, so the address arithmetic of a uniform row base stays
// scalar, and offsets at or beyond `bytes` read zero.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
constexpr int AUX_NT = 2;  // non-temporal (streamed once)
__device__ __forceinline__ v4i buf_ld16(rsrc_t r, uint32_t voff, int soff = 0) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, soff, 0));
}
__device__ __forceinline__ v4i buf_ld16_nt(rsrc_t r, uint32_t voff, int soff = 0) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, soff, AUX_NT));
}

// Raw buffer descriptor in four SGPRs: base, stride 0, num_records = bytes, gfx9 word 3.
__device__ __forceinline__ v4i make_desc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return v4i{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), (int)bytes, 0x00020000};
}
// 16 bytes per lane from buffer offset `voff` straight into LDS at lds_base + 16 * lane (lds_base is passed in M0,
// which the compiler loads for the asm). Written as inline asm so the compiler, which cannot see which LDS bytes
// the load writes, does not drain every outstanding load before each LDS read or barrier; the kernel orders it with
// explicit s_waitcnt + barrier.
// The compiler does not insert wait states in front of an inline-asm statement, and two gfx9 hazards apply to this
// load's scalar operands: a VALU write of an SGPR (v_readlane_b32 restoring a spilled resource, v_readfirstlane_b32)
// needs 5 wait states before a vector memory instruction reads it, and an SALU write of M0 needs 1 before a
// direct-to-LDS load reads it. Without them the load can take the register's old value: a stale resource base
// faulted the GPU in a persistent GEMM whose spilled resource was reloaded just before its load. Hence the
// `s_nop 4` (5 wait states) inside the statement; hazard_lint.py checks the built library for both hazards.
#define LFM2Q_LDS_DMA_WAIT "s_nop 4\n\t"
__device__ __forceinline__ void lds_dma16(v4i desc, uint32_t voff, uint32_t lds_base) {
    asm volatile(LFM2Q_LDS_DMA_WAIT "buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(desc),
                 "{m0}"(lds_base)
                 : "memory");
}
// 4 bytes per lane from buffer offset `voff` into LDS at lds_base + 4 * lane
__device__ __forceinline__ void lds_dma4(v4i desc, uint32_t voff, uint32_t lds_base) {
    asm volatile(LFM2Q_LDS_DMA_WAIT "buffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(desc), "{m0}"(lds_base)
                 : "memory");
}
// The same two loads at device scope (sc1): they do not take a line this XCD's L2 may hold from before, for data
// another XCD's workgroup wrote with device-scope stores during the same launch.
__device__ __forceinline__ void lds_dma16_dev(v4i desc, uint32_t voff, uint32_t lds_base) {
    asm volatile(LFM2Q_LDS_DMA_WAIT "buffer_load_dwordx4 %0, %1, 0 offen sc1 lds" ::"v"(voff), "s"(desc),
                 "{m0}"(lds_base)
                 : "memory");
}
__device__ __forceinline__ void lds_dma4_dev(v4i desc, uint32_t voff, uint32_t lds_base) {
    asm volatile(LFM2Q_LDS_DMA_WAIT "buffer_load_dword %0, %1, 0 offen sc1 lds" ::"v"(voff), "s"(desc),
                 "{m0}"(lds_base)
                 : "memory");
}
// LDS address of p as a wavefront-uniform (SGPR) value for M0
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(p));
}

// SiLU as the reference computes it, silu(g) = g / (1 + exp(-g)) in fp32, on the hardware exp2 and reciprocal:
// exp(-g) = 2^x, x = t log2(e) with t = -g, carried as x_hi + x_lo (the fma residual of the rounded product plus the
// constant's own low part), 2^x_hi on v_exp_f32 times the first-order correction 1 + x_lo ln 2, then d = 1 + exp(-g)
// rounded as the reference rounds it; the quotient g / d from v_rcp_f32 with one fma correction,
// q - (q d - g) r. The edges, each without a branch:
//  - t is clamped to [-128, 128] (v_med3): exp(-g) has rounded to 0 or inf well before, and past |t| ~ 2^24 x_lo is no
//    longer small (the correction factor could turn the overflow negative, and t log2(e) itself overflows near
//    FLT_MAX);
//  - v_rcp_f32 flushes a denormal result, so past d = 2^64 (g < -44) the quotient is formed as (g 2^-64) / (d 2^-64)
//    (exact scalings; the result stays a normal number down to where exp(-g) overflows);
//  - once exp(-g) has overflowed, r = 1/inf = 0 and q = g x 0 = -0, the reference's g / inf; d is capped at 2^64 in
//    the residual so that q d does not become 0 x inf (finite d never reaches the cap after the scaling). g = -inf
//    gives NaN, as g / inf does;
//  - the residual is written q d - g, not g - q d, so that g = -0 keeps its sign through the correction;
//  - g = +inf is the one select (the residual is inf - inf there); the reference gives g / 1.
// Contraction is off so that every rounding is the one written. About 20 VALU instructions against ~25 plus branches
// for the math library's expf and the IEEE division. The callers all round g to bf16 first and the result to bf16
// after; over all 65536 bf16 inputs the result equals the C library's g / (1 + expf(-g)) rounded to bf16.
__device__ __forceinline__ float silu_f32(float g) {
#pragma clang fp contract(off)
    constexpr float L_HI = 1.44269502f, L_LO = 1.92596299e-8f;  // log2(e) = L_HI + L_LO
    const float t = __builtin_amdgcn_fmed3f(-g, -128.f, 128.f);
    const float xh = t * L_HI;
    const float xl = __builtin_fmaf(t, L_LO, __builtin_fmaf(t, L_HI, -xh));
    const float e = __builtin_amdgcn_exp2f(xh) * __builtin_fmaf(xl, 0.693147182f, 1.f);
    const float d = 1.f + e;
    const float sc = d > 0x1p64f ? 0x1p-64f : 1.f;
    const float ds = d * sc, gs = g * sc;
    const float r = __builtin_amdgcn_rcpf(ds);
    const float q = gs * r;
    const float rr = __builtin_fmaf(q, __builtin_fminf(ds, 0x1p64f), -gs);
    const float res = __builtin_fmaf(-rr, r, q);
    return g == __builtin_inff() ? g : res;
}

// GELU, tanh form: 0.5 v (1 + tanh(u)), u = sqrt(2/pi) (v + 0.044715 v^3), with 1 + tanh(u) formed in fp32 as the
// reference forms it (for large negative v that sum cancels, and the result follows it). tanh comes from the identity
// tanh(a) = 1 - 2 / (e^{2a} + 1), a = |u|, sign restored afterwards: e^{2a} = 2^x, x = 2a log2(e) carried as
// x_hi + x_lo (the fma residual of the rounded product plus the constant's own low part), 2^x_hi on v_exp_f32 times
// the first-order correction 1 + x_lo ln 2, and v_rcp_f32 for the reciprocal (each within about an ulp). a is capped
// at 16, where tanh already rounds to 1 in fp32: past |v| ~ 7e12 the cube overflows, u is inf and x_lo would be
// inf - inf. Near u = 0 the identity gives tanh only to ~1e-7 absolute -- not tanh's full relative accuracy there,
// but 1 + tanh(u) is all the GELU uses, and that stays within an ulp or two. About 16 VALU instructions, against ~38
// for the math library's tanhf with its small-argument polynomial and range checks (the GELU epilogue dominated the
// GELU GEMMs).
__device__ __forceinline__ float gelu_tanh_f32(float v) {
    const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    const float a = __builtin_fminf(__builtin_fabsf(u), 16.f);
    constexpr float C_HI = 2.88539004f, C_LO = 3.85192598e-8f;  // 2 log2(e) = C_HI + C_LO
    const float xh = a * C_HI;
    const float xl = __builtin_fmaf(a, C_HI, -xh) + a * C_LO;
    const float e = __builtin_amdgcn_exp2f(xh) * __builtin_fmaf(xl, 0.693147182f, 1.f);  // e^{2a}
    const float t = __builtin_fmaf(-2.f, __builtin_amdgcn_rcpf(e + 1.f), 1.f);            // tanh(a)
    return 0.5f * v * (1.f + __builtin_copysignf(t, u));
}

}  // namespace lfm2q
