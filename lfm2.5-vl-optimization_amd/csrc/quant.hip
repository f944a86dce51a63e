// Activation quantization for the W8A8 GEMM on gfx950 and the fused producers that emit its INT8 input directly:
//   quant_rows      s = max(amax, 1e-8) / 127 per row,            q = rint(x / s)
//   quant_groups    the same per row and group of 64 columns, scales written transposed sT[K/64][rows]
//   add_rmsnorm_q   h = bf16(h + y); x = bf16(w * bf16(h * rsqrt(mean(h^2) + eps)))           -> quantized x
//   add_layernorm_q h = bf16(h + y); x = bf16(((h - mean) * rstd) * w + b)                    -> quantized x
//   silu_mul_q      x = bf16(bf16(silu(g1)) * g3) on g = [g1 | g3], exactly lfm2q_silu_mul's -> quantized x
// One wavefront per row, the row in registers: lane l holds the 16-byte vectors c * 64 + l (c < CH, 8 bf16 each) of
// the row, so a row of up to 8192 values takes one read and one write. Every producer can also write its bf16 x:
// the INT8 output is then bit-identical to quant_rows / quant_groups of that x (the same quantizer code runs on the
// same bf16 values), which is the reference's own test of the fused kernels.
//
// Reference: kernels/int8_gemm.cu:391-474 (quant_rows_kernel, quant_groups_kernel), :491-682 (warp_quant_store,
// add_layernorm_q_kernel, add_rmsnorm_q_kernel, silu_mul_q_kernel); bf16 forms kernels/lfm2_decode.cu:96-121
// (add_rmsnorm), kernels/vision_ops.cu:29-80 (add_layernorm); bound in kernels/int8_gemm.cpp:83-141.
#include "common.hpp"
#include "quantize.hpp"
#include "rmsnorm.hpp"
#include "status.hpp"

#include <algorithm>

namespace lfm2q {
namespace {

// Quantize one row held as above (C = vectors in the row; lanes past it hold zeros) into qr and its scale(s):
// GROUPED = false: one scale s[row]; true: one scale per 64 columns, i.e. per 8 consecutive lanes of a vector index
// c, written to s[g * rows + row] (g = the group's index in the row).
template <int CH, bool GROUPED>
__device__ __forceinline__ void quant_store(const v4i (&v)[CH], int C, int8_t *__restrict__ qr, float *__restrict__ s,
                                            int row, int rows, int lane) {
    float sc_row = 0.f, rc_row = 0.f;
    if (!GROUPED) {
        float m = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) m = absmax8(v[c], m);
        sc_row = scale_of(wave_max(m));
        rc_row = 1.f / sc_row;
        if (lane == 0) s[row] = sc_row;
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 64 + lane;
        float sc = sc_row, rc = rc_row;
        if (GROUPED) {
            float m = absmax8(v[c], 0.f);
            m = fmaxf(m, __shfl_xor(m, 1));
            m = fmaxf(m, __shfl_xor(m, 2));
            m = fmaxf(m, __shfl_xor(m, 4));
            sc = scale_of(m);
            rc = 1.f / sc;
            if (i < C && (lane & 7) == 0) s[(size_t)(i >> 3) * rows + row] = sc;
        }
        if (i < C) {
            int lo, hi;
            quant8(v[c], sc, rc, lo, hi);
            *reinterpret_cast<int2 *>(qr + (size_t)i * 8) = make_int2(lo, hi);
        }
    }
}

__device__ __forceinline__ int row_of_wave() {
    return __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
}

// ------------------------------------------------------------------------------------------------ quant_rows / groups
// CH > 0: K <= 512 CH, the row in registers. CH == 0: longer rows; per-row scales take two passes over the row (the
// second one hits the cache), grouped scales one (64 lanes x one vector = 8 whole groups per step).
template <int CH, bool GROUPED>
__global__ __launch_bounds__(256) void quant_kernel(const uint16_t *__restrict__ x, int8_t *__restrict__ q,
                                                    float *__restrict__ s, int rows, int K) {
    const int lane = threadIdx.x & 63;
    const int row = row_of_wave();
    if (row >= rows) return;
    const uint16_t *xr = x + (size_t)row * K;
    int8_t *qr = q + (size_t)row * K;
    const int C = K / 8;
    if constexpr (CH > 0) {
        v4i v[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i = c * 64 + lane;
            v[c] = i < C ? ld_nt16(xr + (size_t)i * 8) : v4i{0, 0, 0, 0};
        }
        quant_store<CH, GROUPED>(v, C, qr, s, row, rows, lane);
    } else if constexpr (GROUPED) {
        for (int c0 = 0; c0 < C; c0 += 64) {
            const int i = c0 + lane;
            const v4i v[1] = {i < C ? ld16(xr + (size_t)i * 8) : v4i{0, 0, 0, 0}};
            quant_store<1, true>(v, C - c0, qr + (size_t)c0 * 8, s + (size_t)(c0 >> 3) * rows, row, rows, lane);
        }
    } else {
        float m = 0.f;
        for (int c = lane; c < C; c += 64) m = absmax8(ld16(xr + (size_t)c * 8), m);
        const float sc = scale_of(wave_max(m)), rc = 1.f / sc;
        if (lane == 0) s[row] = sc;
        for (int c = lane; c < C; c += 64) {
            int lo, hi;
            quant8(ld16(xr + (size_t)c * 8), sc, rc, lo, hi);
            *reinterpret_cast<int2 *>(qr + (size_t)c * 8) = make_int2(lo, hi);
        }
    }
}

// One row per workgroup of 4 wavefronts, for the shapes where one wavefront per row leaves the CUs short of
// wavefronts (few rows) or makes each one long (K up to 8192: 16 vectors per lane, ~1300 VALU instructions of
// quantization per wavefront): thread t (0 .. 255) holds the vectors c 256 + t (c < CH) of the row. Per-row scales
// take the wavefronts' maxima through LDS (a maximum does not depend on the order it is taken in); a grouped scale
// covers 8 consecutive vectors, i.e. 8 consecutive lanes of one wavefront, as in quant_kernel. Each value is quantized
// by the same quant8 with the same scale and reciprocal, so the bytes and scales equal quant_kernel's.
// Quantize one row held by a workgroup's 256 threads (thread t: vectors c 256 + t, c < CH; threads past the row hold
// zeros) into qr and its scale(s), as quant_store does for a row held by one wavefront.
template <int CH, bool GROUPED>
__device__ __forceinline__ void quant_store_wg(const v4i (&v)[CH], int C, int8_t *__restrict__ qr,
                                               float *__restrict__ s, int row, int rows, int t) {
    const int lane = t & 63, wave = t >> 6;
    float sc_row = 0.f, rc_row = 0.f;
    if (!GROUPED) {
        __shared__ float wmax[4];
        float m = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) m = absmax8(v[c], m);
        m = wave_max(m);
        if (lane == 0) wmax[wave] = m;
        __syncthreads();
        sc_row = scale_of(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
        rc_row = 1.f / sc_row;
        if (t == 0) s[row] = sc_row;
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 256 + t;
        float sc = sc_row, rc = rc_row;
        if (GROUPED) {
            float m = absmax8(v[c], 0.f);
            m = fmaxf(m, __shfl_xor(m, 1));
            m = fmaxf(m, __shfl_xor(m, 2));
            m = fmaxf(m, __shfl_xor(m, 4));
            sc = scale_of(m);
            rc = 1.f / sc;
            if (i < C && (t & 7) == 0) s[(size_t)(i >> 3) * rows + row] = sc;
        }
        if (i < C) {
            int lo, hi;
            quant8(v[c], sc, rc, lo, hi);
            *reinterpret_cast<int2 *>(qr + (size_t)i * 8) = make_int2(lo, hi);
        }
    }
}

template <int CH, bool GROUPED>
__global__ __launch_bounds__(256) void quant_row_wg_kernel(const uint16_t *__restrict__ x, int8_t *__restrict__ q,
                                                           float *__restrict__ s, int rows, int K) {
    const int t = threadIdx.x;
    const int row = blockIdx.x;
    const uint16_t *xr = x + (size_t)row * K;
    const int C = K / 8;
    v4i v[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 256 + t;
        v[c] = i < C ? ld_nt16(xr + (size_t)i * 8) : v4i{0, 0, 0, 0};
    }
    quant_store_wg<CH, GROUPED>(v, C, q + (size_t)row * K, s, row, rows, t);
}

// Per-row scales only, s = max(amax, 1e-8) / 127 -- the s of quant_rows (a maximum does not depend on the order it
// is taken in): the first pass of the bf16-activation GEMM, which quantizes the rows itself with these scales.
__global__ __launch_bounds__(256) void row_scale_kernel(const uint16_t *__restrict__ x, float *__restrict__ s, int rows,
                                                        int K) {
    const int lane = threadIdx.x & 63;
    const int row = row_of_wave();
    if (row >= rows) return;
    const uint16_t *xr = x + (size_t)row * K;
    float m = 0.f;
    for (int c = lane; c < K / 8; c += 64) m = absmax8(ld16(xr + (size_t)c * 8), m);
    m = wave_max(m);
    if (lane == 0) s[row] = scale_of(m);
}

// ------------------------------------------------------------------------------------------------ producers

// row (+ residual) -> registers. ADD: h = bf16(h + y), written back. Lanes past the row get zeros. Every load is
// issued before the first use -- a lane past the row reads the row's last chunk and drops it -- so the row costs one
// memory round trip whatever CH (a row per wavefront is latency-bound when there are few rows, as in decoding).
template <int CH>
__device__ __forceinline__ void load_row_add(uint16_t *__restrict__ hr, const uint16_t *__restrict__ yr, int C,
                                             int lane, v4i (&hv)[CH]) {
    v4i yv[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const size_t o = (size_t)min(c * 64 + lane, C - 1) * 8;
        hv[c] = ld16(hr + o);
        if (yr) yv[c] = ld16(yr + o);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 64 + lane;
        if (i >= C) {
            hv[c] = v4i{0, 0, 0, 0};
        } else if (yr) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                hv[c][j] = (int)pack_bf16x2(bf2f_lo((uint32_t)hv[c][j]) + bf2f_lo((uint32_t)yv[c][j]),
                                      bf2f_hi((uint32_t)hv[c][j]) + bf2f_hi((uint32_t)yv[c][j]));
            *reinterpret_cast<v4i *>(hr + (size_t)i * 8) = hv[c];
        }
    }
}

// a per-column parameter vector (norm weight / bias) of the row's layout, loaded up front like the row
template <int CH>
__device__ __forceinline__ void load_params(const uint16_t *__restrict__ p, int C, int lane, v4i (&pv)[CH]) {
#pragma unroll
    for (int c = 0; c < CH; ++c) pv[c] = ld16(p + (size_t)min(c * 64 + lane, C - 1) * 8);
}

template <int CH>
__device__ __forceinline__ void store_row(uint16_t *__restrict__ xr, const v4i (&xv)[CH], int C, int lane) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 64 + lane;
        if (i < C) *reinterpret_cast<v4i *>(xr + (size_t)i * 8) = xv[c];
    }
}

template <int CH, bool GROUPED>
__global__ __launch_bounds__(256) void add_rmsnorm_q_kernel(uint16_t *__restrict__ h, const uint16_t *__restrict__ y,
                                                            const uint16_t *__restrict__ w, int8_t *__restrict__ q,
                                                            float *__restrict__ s, uint16_t *__restrict__ xo, int rows,
                                                            int H, float eps) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int row = row_of_wave();
    if (row >= rows) return;
    const int C = H / 8;
    v4i wv[CH], hv[CH];
    load_params<CH>(w, C, lane, wv);  // in flight with the row, used after the reduction
    load_row_add<CH>(h + (size_t)row * H, y ? y + (size_t)row * H : nullptr, C, lane, hv);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) ss = sumsq8(hv[c], ss);
    const float rs = rms_scale(wave_sum(ss), H, eps);
    v4i xv[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 64 + lane;
        xv[c] = v4i{0, 0, 0, 0};
        if (i < C) {
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[c][j] = (int)rms_apply2((uint32_t)wv[c][j], (uint32_t)hv[c][j], rs);
        }
    }
    if (xo) store_row<CH>(xo + (size_t)row * H, xv, C, lane);
    quant_store<CH, GROUPED>(xv, C, q + (size_t)row * H, s, row, rows, lane);
}

// add_rmsnorm_q for rows of at most 64 values (the per-head q / k norms of head_dim 64): eight rows per wavefront,
// lane 8 r + j holding vector j (j < C) of row r, where one wavefront per row would leave 56 of its 64 lanes idle.
// The sum of squares is folded by the steps of wave_sum that stay within 8 lanes (DPP xor 1, xor 2, half mirror);
// with one wavefront per row wave_sum's remaining steps add only the zeros of the lanes past the row, so each row
// gets add_rmsnorm_q_kernel's bits. The row maximum is taken over the row's 8 lanes (order-free), and with H = 64 a
// row is one 64-column group, so per-row and grouped scales are the same value in the same slot s[row].
__global__ __launch_bounds__(256) void add_rmsnorm_q_short_kernel(uint16_t *__restrict__ h,
                                                                  const uint16_t *__restrict__ y,
                                                                  const uint16_t *__restrict__ w,
                                                                  int8_t *__restrict__ q, float *__restrict__ s,
                                                                  uint16_t *__restrict__ xo, int rows, int H,
                                                                  float eps) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
    const int j = lane & 7, C = H / 8;
    const bool act = row < rows && j < C;  // every lane takes part in the lane exchanges below
    const size_t o = (size_t)row * H + (size_t)j * 8;
    v4i hv = {0, 0, 0, 0}, yv = {0, 0, 0, 0}, wv = {0, 0, 0, 0};
    if (act) {
        hv = ld16(h + o);
        if (y) yv = ld16(y + o);
        wv = ld16(w + (size_t)j * 8);
    }
    if (act && y) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            hv[k] = (int)pack_bf16x2(bf2f_lo((uint32_t)hv[k]) + bf2f_lo((uint32_t)yv[k]),
                                     bf2f_hi((uint32_t)hv[k]) + bf2f_hi((uint32_t)yv[k]));
        *reinterpret_cast<v4i *>(h + o) = hv;
    }
    float ss = sumsq8(hv, 0.f);
    ss += dpp<DPP_XOR1>(ss);
    ss += dpp<DPP_XOR2>(ss);
    ss += dpp<DPP_HALF_MIRROR>(ss);
    const float rs = rms_scale(ss, H, eps);
    v4i xv = {0, 0, 0, 0};
    if (act) {
#pragma unroll
        for (int k = 0; k < 4; ++k) xv[k] = (int)rms_apply2((uint32_t)wv[k], (uint32_t)hv[k], rs);
        if (xo) *reinterpret_cast<v4i *>(xo + o) = xv;
    }
    float m = absmax8(xv, 0.f);
    m = fmaxf(m, dpp<DPP_XOR1>(m));
    m = fmaxf(m, dpp<DPP_XOR2>(m));
    m = fmaxf(m, dpp<DPP_HALF_MIRROR>(m));
    const float sc = scale_of(m), rc = 1.f / sc;
    if (act) {
        int lo, hi;
        quant8(xv, sc, rc, lo, hi);
        *reinterpret_cast<int2 *>(q + o) = make_int2(lo, hi);
        if (j == 0) s[row] = sc;
    }
}

template <int CH, bool GROUPED>
__global__ __launch_bounds__(256) void add_layernorm_q_kernel(uint16_t *__restrict__ h,
                                                              const uint16_t *__restrict__ y,
                                                              const uint16_t *__restrict__ w,
                                                              const uint16_t *__restrict__ b, int8_t *__restrict__ q,
                                                              float *__restrict__ s, uint16_t *__restrict__ xo,
                                                              int rows, int D, float eps) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int row = row_of_wave();
    if (row >= rows) return;
    const int C = D / 8;
    v4i wv[CH], bv[CH], hv[CH];
    load_params<CH>(w, C, lane, wv);  // in flight with the row, used after the reductions
    load_params<CH>(b, C, lane, bv);
    load_row_add<CH>(h + (size_t)row * D, y ? y + (size_t)row * D : nullptr, C, lane, hv);
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) sum += bf2f_lo((uint32_t)hv[c][j]) + bf2f_hi((uint32_t)hv[c][j]);
    const float mean = wave_sum(sum) / (float)D;
    float qs = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        if (c * 64 + lane < C) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float a = bf2f_lo((uint32_t)hv[c][j]) - mean, d = bf2f_hi((uint32_t)hv[c][j]) - mean;
                qs += a * a;
                qs += d * d;
            }
        }
    }
    const float rstd = 1.f / sqrtf(wave_sum(qs) / (float)D + eps);
    v4i xv[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 64 + lane;
        xv[c] = v4i{0, 0, 0, 0};
        if (i < C) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = ((bf2f_lo((uint32_t)hv[c][j]) - mean) * rstd) * bf2f_lo((uint32_t)wv[c][j]);
                const float hi = ((bf2f_hi((uint32_t)hv[c][j]) - mean) * rstd) * bf2f_hi((uint32_t)wv[c][j]);
                xv[c][j] = (int)pack_bf16x2(lo + bf2f_lo((uint32_t)bv[c][j]), hi + bf2f_hi((uint32_t)bv[c][j]));
            }
        }
    }
    if (xo) store_row<CH>(xo + (size_t)row * D, xv, C, lane);
    quant_store<CH, GROUPED>(xv, C, q + (size_t)row * D, s, row, rows, lane);
}

template <int CH, bool GROUPED>
__global__ __launch_bounds__(256) void silu_mul_q_kernel(const uint16_t *__restrict__ g, int8_t *__restrict__ q,
                                                         float *__restrict__ s, uint16_t *__restrict__ xo, int rows,
                                                         int I) {
    const int lane = threadIdx.x & 63;
    const int row = row_of_wave();
    if (row >= rows) return;
    const int C = I / 8;
    const uint16_t *gr = g + (size_t)row * 2 * I;
    v4i xv[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 64 + lane;
        xv[c] = v4i{0, 0, 0, 0};
        if (i < C) {
            const v4i av = ld_nt16(gr + (size_t)i * 8), uv = ld_nt16(gr + I + (size_t)i * 8);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[c][j] = (int)pack_bf16x2(rbf(silu_f32(bf2f_lo((uint32_t)av[j]))) * bf2f_lo((uint32_t)uv[j]),
                                      rbf(silu_f32(bf2f_hi((uint32_t)av[j]))) * bf2f_hi((uint32_t)uv[j]));
        }
    }
    if (xo) store_row<CH>(xo + (size_t)row * I, xv, C, lane);
    quant_store<CH, GROUPED>(xv, C, q + (size_t)row * I, s, row, rows, lane);
}

// silu_mul_q with a workgroup per row (long rows: I = 8192 holds 128 values per lane on one wavefront, 171 VGPRs,
// two wavefronts per SIMD, each running its loads, ~30 VALU per value of SiLU and quantization, and its stores in
// turn): thread t holds the vectors c 256 + t (c < CH), every load issued before the first SiLU, then
// quant_store_wg. Each value is the same expression as silu_mul_q_kernel's and the row / group maxima do not depend
// on the order they are taken in, so the bytes, scales and bf16 x are the same.
template <int CH, bool GROUPED>
__global__ __launch_bounds__(256) void silu_mul_q_wg_kernel(const uint16_t *__restrict__ g, int8_t *__restrict__ q,
                                                            float *__restrict__ s, uint16_t *__restrict__ xo,
                                                            int rows, int I) {
    const int t = threadIdx.x;
    const int row = blockIdx.x;
    const int C = I / 8;
    const uint16_t *gr = g + (size_t)row * 2 * I;
    v4i av[CH], uv[CH], xv[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 256 + t;
        if (i < C) {
            av[c] = ld_nt16(gr + (size_t)i * 8);
            uv[c] = ld_nt16(gr + I + (size_t)i * 8);
        }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 256 + t;
        xv[c] = v4i{0, 0, 0, 0};
        if (i < C) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[c][j] = (int)pack_bf16x2(rbf(silu_f32(bf2f_lo((uint32_t)av[c][j]))) * bf2f_lo((uint32_t)uv[c][j]),
                                      rbf(silu_f32(bf2f_hi((uint32_t)av[c][j]))) * bf2f_hi((uint32_t)uv[c][j]));
            if (xo) *reinterpret_cast<v4i *>(xo + (size_t)row * I + (size_t)i * 8) = xv[c];
        }
    }
    quant_store_wg<CH, GROUPED>(xv, C, q + (size_t)row * I, s, row, rows, t);
}

// ------------------------------------------------------------------------------------------------ dispatch
// CH = vectors of 8 per lane holding a row of `len` values: len <= 512 CH <= 8192
#define LFM2Q_CH_SWITCH(len, CALL)                                                                                  \
    switch (((len) + 511) / 512) {                                                                                   \
        case 1: CALL(1); break;                                                                                      \
        case 2: CALL(2); break;                                                                                      \
        case 3: CALL(3); break;                                                                                      \
        case 4: CALL(4); break;                                                                                      \
        case 5: CALL(5); break;                                                                                      \
        case 6: CALL(6); break;                                                                                      \
        case 7: CALL(7); break;                                                                                      \
        case 8: CALL(8); break;                                                                                      \
        case 9: CALL(9); break;                                                                                      \
        case 10: CALL(10); break;                                                                                    \
        case 11: CALL(11); break;                                                                                    \
        case 12: CALL(12); break;                                                                                    \
        case 13: CALL(13); break;                                                                                    \
        case 14: CALL(14); break;                                                                                    \
        case 15: CALL(15); break;                                                                                    \
        default: CALL(16); break;                                                                                    \
    }

// quant_rows / quant_groups launch: a workgroup per row (quant_row_wg_kernel) or a wavefront per row (quant_kernel).
// Knob LFM2Q_QUANT_WG: 1 / 0 forces one or the other. Default, from MI355X timings of both forms on the W8A8
// workload's activations (bench.py --quant-sweep): a workgroup per row from K = 4096 (512 x 8192 12.6 -> 6.4 us,
// 4096 x 8192 31.7 -> 20.6 us, 10240 x 4304 31.2 -> 27.9 us), and from K = 2048 with grouped scales or at most
// 8 rows per CU (512 x 2048 4.6 -> 3.3 us); a wavefront per row for the short vision rows (10240 x 1152: 10.9 against
// 14.3 us, half of a workgroup's threads would hold no vector) and for many per-token rows of 2048.
inline bool wg_rows(int rows, int K, bool grouped) {
    const int f = knob_int(KNOB_QUANT_WG, -1);
    if (K > 8192) return false;
    if (f >= 0) return f != 0;
    return K >= 4096 || (K >= 2048 && (grouped || rows <= 8 * device_cus()));
}

template <bool GROUPED>
void launch_quant(const uint16_t *x, int8_t *q, float *s, int rows, int K, hipStream_t st) {
    if (wg_rows(rows, K, GROUPED)) {
        const int C = K / 8;
        switch ((C + 255) / 256) {
            case 1: quant_row_wg_kernel<1, GROUPED><<<rows, 256, 0, st>>>(x, q, s, rows, K); break;
            case 2: quant_row_wg_kernel<2, GROUPED><<<rows, 256, 0, st>>>(x, q, s, rows, K); break;
            case 3: quant_row_wg_kernel<3, GROUPED><<<rows, 256, 0, st>>>(x, q, s, rows, K); break;
            default: quant_row_wg_kernel<4, GROUPED><<<rows, 256, 0, st>>>(x, q, s, rows, K); break;
        }
        return;
    }
    const dim3 grid((rows + 3) / 4);
#define LFM2Q_Q(CH_) quant_kernel<CH_, GROUPED><<<grid, 256, 0, st>>>(x, q, s, rows, K)
    if (K > 8192)
        LFM2Q_Q(0);
    else
        LFM2Q_CH_SWITCH(K, LFM2Q_Q)
#undef LFM2Q_Q
}

int check_rows(const char *name, int rows, int len, int grouped, int maxlen) {
    LFM2Q_REQUIRE(rows >= 1 && len >= 8, LFM2Q_ERR_SHAPE, "%s: need rows >= 1 and a row length >= 8 (rows=%d, %d)",
                  name, rows, len);
    LFM2Q_REQUIRE(len % (grouped ? 64 : 8) == 0, LFM2Q_ERR_SHAPE, "%s: row length must be a multiple of %d (%d)", name,
                  grouped ? 64 : 8, len);
    LFM2Q_REQUIRE(len <= maxlen, LFM2Q_ERR_SHAPE, "%s: row length must be <= %d (%d)", name, maxlen, len);
    return LFM2Q_OK;
}

}  // namespace

int launch_row_scales(const uint16_t *x, float *s, int rows, int K, hipStream_t st) {
    row_scale_kernel<<<(rows + 3) / 4, 256, 0, st>>>(x, s, rows, K);
    return launch_status("row scales");
}

}  // namespace lfm2q

using namespace lfm2q;

extern "C" int lfm2q_quant_rows(const lfm2q_bf16 *x, int8_t *q, float *s, int rows, int K, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(x && q && s, LFM2Q_ERR_ARG, "quant_rows: null pointer");
    LFM2Q_REQUIRE(rows >= 1 && K >= 8 && K % 8 == 0, LFM2Q_ERR_SHAPE,
                  "quant_rows: K must be a multiple of 8 (rows=%d K=%d)", rows, K);
    LFM2Q_REQUIRE(aligned16(x) && ((uintptr_t)q & 7) == 0, LFM2Q_ERR_ALIGN,
                  "quant_rows: x must be 16-byte and q 8-byte aligned");
    launch_quant<false>(x, q, s, rows, K, (hipStream_t)stream);
    return launch_status("quant_rows");
}

extern "C" int lfm2q_quant_groups(const lfm2q_bf16 *x, int8_t *q, float *sT, int rows, int K, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(x && q && sT, LFM2Q_ERR_ARG, "quant_groups: null pointer");
    LFM2Q_REQUIRE(rows >= 1 && K >= 64 && K % 64 == 0, LFM2Q_ERR_SHAPE,
                  "quant_groups: K must be a multiple of 64 (rows=%d K=%d)", rows, K);
    LFM2Q_REQUIRE(aligned16(x) && ((uintptr_t)q & 7) == 0, LFM2Q_ERR_ALIGN,
                  "quant_groups: x must be 16-byte and q 8-byte aligned");
    launch_quant<true>(x, q, sT, rows, K, (hipStream_t)stream);
    return launch_status("quant_groups");
}

extern "C" int lfm2q_add_rmsnorm_q(lfm2q_bf16 *h, const lfm2q_bf16 *y, const lfm2q_bf16 *w, int8_t *q, float *s,
                                   lfm2q_bf16 *x, int rows, int H, float eps, int grouped, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(h && w && q && s, LFM2Q_ERR_ARG, "add_rmsnorm_q: null pointer");
    if (int st = check_rows("add_rmsnorm_q", rows, H, grouped, 8192)) return st;
    LFM2Q_REQUIRE(aligned16(h) && aligned16(w) && (!y || aligned16(y)) && (!x || aligned16(x)) && ((uintptr_t)q & 7) == 0,
                  LFM2Q_ERR_ALIGN, "add_rmsnorm_q: h, y, w, x must be 16-byte and q 8-byte aligned");
    const dim3 grid((rows + 3) / 4);
    const hipStream_t st = (hipStream_t)stream;
    if (H <= 64 && knob_int(KNOB_QUANT_WG, -1) != 0) {  // short rows: eight per wavefront (knob 0: one per wavefront)
        add_rmsnorm_q_short_kernel<<<(rows + 31) / 32, 256, 0, st>>>(h, y, w, q, s, x, rows, H, eps);
        return launch_status("add_rmsnorm_q");
    }
#define LFM2Q_P(CH_)                                                                                                 \
    if (grouped)                                                                                                     \
        add_rmsnorm_q_kernel<CH_, true><<<grid, 256, 0, st>>>(h, y, w, q, s, x, rows, H, eps);                       \
    else                                                                                                             \
        add_rmsnorm_q_kernel<CH_, false><<<grid, 256, 0, st>>>(h, y, w, q, s, x, rows, H, eps)
    LFM2Q_CH_SWITCH(H, LFM2Q_P)
#undef LFM2Q_P
    return launch_status("add_rmsnorm_q");
}

extern "C" int lfm2q_add_layernorm_q(lfm2q_bf16 *h, const lfm2q_bf16 *y, const lfm2q_bf16 *w, const lfm2q_bf16 *b,
                                     int8_t *q, float *s, lfm2q_bf16 *x, int rows, int D, float eps, int grouped,
                                     lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(h && w && b && q && s, LFM2Q_ERR_ARG, "add_layernorm_q: null pointer");
    if (int st = check_rows("add_layernorm_q", rows, D, grouped, 8192)) return st;
    LFM2Q_REQUIRE(aligned16(h) && aligned16(w) && aligned16(b) && (!y || aligned16(y)) && (!x || aligned16(x)) &&
                      ((uintptr_t)q & 7) == 0,
                  LFM2Q_ERR_ALIGN, "add_layernorm_q: h, y, w, b, x must be 16-byte and q 8-byte aligned");
    const dim3 grid((rows + 3) / 4);
    const hipStream_t st = (hipStream_t)stream;
#define LFM2Q_P(CH_)                                                                                                 \
    if (grouped)                                                                                                     \
        add_layernorm_q_kernel<CH_, true><<<grid, 256, 0, st>>>(h, y, w, b, q, s, x, rows, D, eps);                  \
    else                                                                                                             \
        add_layernorm_q_kernel<CH_, false><<<grid, 256, 0, st>>>(h, y, w, b, q, s, x, rows, D, eps)
    LFM2Q_CH_SWITCH(D, LFM2Q_P)
#undef LFM2Q_P
    return launch_status("add_layernorm_q");
}

extern "C" int lfm2q_silu_mul_q(const lfm2q_bf16 *g, int8_t *q, float *s, lfm2q_bf16 *x, int rows, int I, int grouped,
                                lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(g && q && s, LFM2Q_ERR_ARG, "silu_mul_q: null pointer");
    if (int st = check_rows("silu_mul_q", rows, I, grouped, 8192)) return st;
    LFM2Q_REQUIRE(aligned16(g) && (!x || aligned16(x)) && ((uintptr_t)q & 7) == 0, LFM2Q_ERR_ALIGN,
                  "silu_mul_q: g, x must be 16-byte and q 8-byte aligned");
    const dim3 grid((rows + 3) / 4);
    const hipStream_t st = (hipStream_t)stream;
    // a workgroup per row from I = 2048 (MI355X, per call over rotating inputs, wavefront -> workgroup form: 4096 x
    // 8192 54.7 -> 41.3 us, grouped 46.9 -> 43.6; 2048 x 8192 29.3 -> 25.8; 512 x 8192 22.5 -> 10.1; 10240 x 4304
    // 57.5 -> 52.9; 4096 x 2048 13.0 -> 12.4, grouped 14.1 -> 12.7); the LFM2Q_QUANT_WG knob forces either form
    const int fwg = knob_int(KNOB_QUANT_WG, -1);
    if (fwg >= 0 ? fwg != 0 : I >= 2048) {
#define LFM2Q_W(CH_)                                                                                                 \
    if (grouped)                                                                                                     \
        silu_mul_q_wg_kernel<CH_, true><<<rows, 256, 0, st>>>(g, q, s, x, rows, I);                                  \
    else                                                                                                             \
        silu_mul_q_wg_kernel<CH_, false><<<rows, 256, 0, st>>>(g, q, s, x, rows, I)
        switch ((I / 8 + 255) / 256) {
            case 1: LFM2Q_W(1); break;
            case 2: LFM2Q_W(2); break;
            case 3: LFM2Q_W(3); break;
            default: LFM2Q_W(4); break;
        }
#undef LFM2Q_W
        return launch_status("silu_mul_q");
    }
#define LFM2Q_P(CH_)                                                                                                 \
    if (grouped)                                                                                                     \
        silu_mul_q_kernel<CH_, true><<<grid, 256, 0, st>>>(g, q, s, x, rows, I);                                     \
    else                                                                                                             \
        silu_mul_q_kernel<CH_, false><<<grid, 256, 0, st>>>(g, q, s, x, rows, I)
    LFM2Q_CH_SWITCH(I, LFM2Q_P)
#undef LFM2Q_P
    return launch_status("silu_mul_q");
}
