// Decode GEMVs for gfx950: y[b, n] = (sum_k W[n, k] x[b, k]) * scale[n] with int8 (weight-only) or bf16 weights,
// bf16 activations, fp32 accumulation, and optional fused SwiGLU / residual-add epilogues.
//
// Two kernels, both pure HBM streams over W (every weight byte is read exactly once per call):
//   gemv_b1_kernel    batch 1. One wavefront owns R output rows; lane l streams the 16-byte chunks l, l+64, ...
//                     of each row with non-temporal loads (a wavefront load = 1 KiB contiguous of one row), all of
//                     a lane's chunks are in flight before the first FMA. int8 -> fp32 is one SDWA convert per
//                     weight; the row sum is a wave64 butterfly. No LDS.
//   gemv_mfma_kernel  batch 2..16. A workgroup owns 16 output rows; its NWK wavefronts split K. Each lane loads
//                     16 weights of one row (row = lane % 16, k-quarter = lane / 16), converts them exactly to
//                     bf16 in registers and feeds v_mfma_f32_16x16x32_bf16 with the activations as the A operand
//                     (16 batch rows x 32 k) and the weights as B (32 k x 16 output rows). The NWK partial 16x16
//                     tiles meet in LDS. The matrix cores take the batch FMAs off the VALU, so the kernel stays
//                     HBM-bound at B = 16, where a VALU GEMV would need 17 VALU ops per weight.
// The per-row accumulation order of each kernel does not depend on which epilogue runs or on how many rows a
// wavefront owns, so the fused epilogues are bit-identical to the plain GEMV followed by the separate op.
//
// Reference: kernels/lfm2_decode.cu:429-950 (gemv_direct_kernel :576-661, gemv_epi_kernel :724-805,
// gemv_dispatch :667-706), kernels/lfm2_decode.cu:954-963 (silu_mul), :108-113 (residual rounding).
#include "common.hpp"
#include "status.hpp"

namespace lfm2q {
namespace {

enum Epi { EPI_NONE = 0, EPI_SWIGLU = 1, EPI_RESIDUAL = 2 };

// ------------------------------------------------------------------------------------------------ chunk math
template <typename WT>
struct Chunk;

template <>
struct Chunk<int8_t> {
    static constexpr int PER = 16;  // weights per 16-byte chunk
    // acc + sum_j w_j x_j over the chunk, summed in element order into a chunk-local partial first
    __device__ static float dot(v4i c, const float *xv, float acc) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = c[j];
            a = fmaf((float)(int8_t)d, xv[4 * j + 0], a);
            a = fmaf((float)(int8_t)(d >> 8), xv[4 * j + 1], a);
            a = fmaf((float)(int8_t)(d >> 16), xv[4 * j + 2], a);
            a = fmaf((float)(d >> 24), xv[4 * j + 3], a);
        }
        return acc + a;
    }
};

template <>
struct Chunk<uint16_t> {  // bf16 weights
    static constexpr int PER = 8;
    __device__ static float dot(v4i c, const float *xv, float acc) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = (uint32_t)c[j];
            a = fmaf(bf2f_lo(d), xv[2 * j], a);
            a = fmaf(bf2f_hi(d), xv[2 * j + 1], a);
        }
        return acc + a;
    }
};

// the PER activations of chunk c of row x (cached loads: x is small and shared by all wavefronts)
template <int PER>
__device__ __forceinline__ void load_x(const uint16_t *__restrict__ x, int c, float *xv) {
    const v4i *p = reinterpret_cast<const v4i *>(x + (size_t)c * PER);
#pragma unroll
    for (int q = 0; q < PER / 8; ++q) {
        const v4i r = p[q];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xv[8 * q + 2 * j] = bf2f_lo((uint32_t)r[j]);
            xv[8 * q + 2 * j + 1] = bf2f_hi((uint32_t)r[j]);
        }
    }
}

__device__ __forceinline__ float apply_scale(float a, const float *__restrict__ scale, int n) {
    return scale ? a * scale[n] : a;
}

// ------------------------------------------------------------------------------------------------ batch 1
// WG = 4 wavefronts; wavefront w of block b owns output rows n0 = (4b + w) R .. n0 + R - 1.
// EPI_SWIGLU: output row n needs weight rows n (w1) and S + n (w3): 2R weight rows per wavefront.
template <typename WT, int R, int U, int EPI>
__global__ __launch_bounds__(256) void gemv_b1_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                      const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                      int N, int K, int S) {
    constexpr int PER = Chunk<WT>::PER;
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 * R : R;
    const int lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (n0 >= N) return;  // no block-level synchronization in this kernel
    const int C = K / PER;
    const char *rp[NROW];
#pragma unroll
    for (int i = 0; i < NROW; ++i) {
        const int orow = min(n0 + (i % R), N - 1);
        const int wrow = (EPI == EPI_SWIGLU && i >= R) ? S + orow : orow;
        rp[i] = reinterpret_cast<const char *>(W + (size_t)wrow * K);
    }
    float acc[NROW];
#pragma unroll
    for (int i = 0; i < NROW; ++i) acc[i] = 0.f;

    for (int c0 = lane; c0 < C; c0 += 64 * U) {
        v4i w[U][NROW];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
#pragma unroll
            for (int i = 0; i < NROW; ++i) w[u][i] = c < C ? ld_nt16(rp[i] + (size_t)c * 16) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
            if (c < C) {
                float xv[PER];
                load_x<PER>(x, c, xv);
#pragma unroll
                for (int i = 0; i < NROW; ++i) acc[i] = Chunk<WT>::dot(w[u][i], xv, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NROW; ++i) acc[i] = wave_sum(acc[i]);

    if (lane >= R) return;
    const int n = n0 + lane;
    if (n >= N) return;
    float a = acc[0], b = EPI == EPI_SWIGLU ? acc[R] : 0.f;
#pragma unroll
    for (int i = 1; i < R; ++i)
        if (lane == i) {
            a = acc[i];
            if (EPI == EPI_SWIGLU) b = acc[R + i];
        }
    if (EPI == EPI_NONE) {
        y[n] = (uint16_t)f2bf(apply_scale(a, scale, n));
    } else if (EPI == EPI_RESIDUAL) {
        y[n] = (uint16_t)f2bf(bf2f(y[n]) + rbf(apply_scale(a, scale, n)));
    } else {
        const float g = rbf(apply_scale(a, scale, n)), u = rbf(apply_scale(b, scale, S + n));
        y[n] = (uint16_t)f2bf(rbf(silu_f32(g)) * u);
    }
}

// ------------------------------------------------------------------------------------------------ batch 2..16
// 8 int8 weights (two dwords) -> 8 bf16 (exact: |q| <= 128 fits the 8-bit bf16 significand)
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    return (__float_as_uint(hi) & 0xffff0000u) | (__float_as_uint(lo) >> 16);
}
__device__ __forceinline__ v8bf i8x8_to_bf16(int d0, int d1) {
    v4u r;
    r[0] = pack_hi16((float)(int8_t)d0, (float)(int8_t)(d0 >> 8));
    r[1] = pack_hi16((float)(int8_t)(d0 >> 16), (float)(d0 >> 24));
    r[2] = pack_hi16((float)(int8_t)d1, (float)(int8_t)(d1 >> 8));
    r[3] = pack_hi16((float)(int8_t)(d1 >> 16), (float)(d1 >> 24));
    return __builtin_bit_cast(v8bf, r);
}
__device__ __forceinline__ v8bf as_bf16x8(v4i v) { return __builtin_bit_cast(v8bf, v); }

// WG = NWK wavefronts, 16 output rows n0..n0+15 (EPI_SWIGLU: 16 rows of w1 and the matching 16 rows of w3).
// Wavefront w covers k in [w K/NWK, (w+1) K/NWK); every step covers 64 k: lane (col = l%16, kq = l/16) loads
// k0 + 16 kq .. +15 of weight row n0 + col and of activation row col (if col < B).
// MFMA layout (v_mfma_f32_16x16x32_bf16): A[i][k] from lane i + 16 (k/8), B[k][j] from lane j + 16 (k/8),
// D[i][j] in lane j + 16 (i/4), element i%4. A and B use the same k <-> (lane group, slot) map, so the product
// pairs x[m][k] with W[n][k] whatever order the hardware sums the 32 k in.
template <typename WT, int NWK, int U, int EPI>
__global__ __launch_bounds__(64 * NWK) void gemv_mfma_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                             const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                             int B, int N, int K, int S) {
    constexpr int NT = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int WL = sizeof(WT) == 1 ? 1 : 2;  // 16-byte weight loads per lane per step
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 15, kq = lane >> 4;
    const int n = blockIdx.x * 16 + col;
    const int nl = min(n, N - 1);
    const WT *wp[NT];
    wp[0] = W + (size_t)nl * K;
    if (EPI == EPI_SWIGLU) wp[NT - 1] = W + (size_t)(S + nl) * K;
    const bool xm = col < B;
    const uint16_t *xp = x + (size_t)(xm ? col : 0) * K;
    const int ks = K / NWK, kb = wave * ks, ke = kb + ks;

    v4f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int k0 = kb; k0 < ke; k0 += 64 * U) {
        v4i wv[U][NT][WL], xv[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + 64 * u + 16 * kq;
            const bool in = k0 + 64 * u < ke;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int h = 0; h < WL; ++h) wv[u][t][h] = in ? ld_nt16(wp[t] + k + 8 * h) : v4i{0, 0, 0, 0};
            xv[u][0] = (in && xm) ? ld16(xp + k) : v4i{0, 0, 0, 0};
            xv[u][1] = (in && xm) ? ld16(xp + k + 8) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (k0 + 64 * u < ke) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    v8bf b0, b1;
                    if (sizeof(WT) == 1) {
                        b0 = i8x8_to_bf16(wv[u][t][0][0], wv[u][t][0][1]);
                        b1 = i8x8_to_bf16(wv[u][t][0][2], wv[u][t][0][3]);
                    } else {
                        b0 = as_bf16x8(wv[u][t][0]);
                        b1 = as_bf16x8(wv[u][t][WL - 1]);
                    }
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xv[u][0]), b0, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xv[u][1]), b1, acc[t], 0, 0, 0);
                }
            }
        }
    }

    if (NWK > 1) {
        __shared__ v4f red[NT][NWK][64];
#pragma unroll
        for (int t = 0; t < NT; ++t) red[t][wave][lane] = acc[t];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            v4f s = red[t][0][lane];
#pragma unroll
            for (int w = 1; w < NWK; ++w) s += red[t][w][lane];
            acc[t] = s;
        }
    }
    if (n >= N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * kq + i;
        if (m >= B) continue;
        const float a = acc[0][i];
        if (EPI == EPI_NONE) {
            y[(size_t)m * N + n] = (uint16_t)f2bf(apply_scale(a, scale, n));
        } else if (EPI == EPI_RESIDUAL) {
            uint16_t *h = y + (size_t)m * N + n;
            *h = (uint16_t)f2bf(bf2f(*h) + rbf(apply_scale(a, scale, n)));
        } else {
            const float g = rbf(apply_scale(a, scale, n)), u = rbf(apply_scale(acc[NT - 1][i], scale, S + n));
            y[(size_t)m * N + n] = (uint16_t)f2bf(rbf(silu_f32(g)) * u);
        }
    }
}

// ------------------------------------------------------------------------------------------------ silu_mul
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ g, uint16_t *__restrict__ y, int I) {
    const int b = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= I) return;
    const float a = bf2f(g[(size_t)b * 2 * I + i]), u = bf2f(g[(size_t)b * 2 * I + I + i]);
    y[(size_t)b * I + i] = (uint16_t)f2bf(rbf(silu_f32(a)) * u);
}

// ------------------------------------------------------------------------------------------------ dispatch
template <typename WT, int R, int EPI>
void launch_b1_u(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int N, int K, int S,
                 hipStream_t st) {
    constexpr int PER = Chunk<WT>::PER;
    const int cpl = (K / PER + 63) / 64;  // chunks per lane
    const dim3 grid((N + 4 * R - 1) / (4 * R));
    if (cpl <= 2)
        gemv_b1_kernel<WT, R, 2, EPI><<<grid, 256, 0, st>>>(W, scale, x, y, N, K, S);
    else if (cpl <= 4)
        gemv_b1_kernel<WT, R, 4, EPI><<<grid, 256, 0, st>>>(W, scale, x, y, N, K, S);
    else
        gemv_b1_kernel<WT, R, 8, EPI><<<grid, 256, 0, st>>>(W, scale, x, y, N, K, S);
}

template <typename WT, int EPI>
void launch_b1(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int N, int K, int S, int rows,
               hipStream_t st) {
    if (EPI == EPI_SWIGLU || rows == 1)
        launch_b1_u<WT, 1, EPI>(W, scale, x, y, N, K, S, st);
    else if (rows == 2)
        launch_b1_u<WT, 2, EPI>(W, scale, x, y, N, K, S, st);
    else
        launch_b1_u<WT, 4, EPI>(W, scale, x, y, N, K, S, st);
}

// wavefronts splitting K: the largest of 8/4/2/1 with at least 512 k per wavefront that divides K into 64-k steps
inline int mfma_nwk(int K) {
    const int steps = K / 64;
    for (int nwk = 8; nwk > 1; nwk >>= 1)
        if (steps % nwk == 0 && K / nwk >= 512) return nwk;
    return 1;
}

template <typename WT, int EPI>
void launch_mfma(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int B, int N, int K, int S,
                 hipStream_t st) {
    const dim3 grid((N + 15) / 16);
    switch (mfma_nwk(K)) {
        case 8: gemv_mfma_kernel<WT, 8, 4, EPI><<<grid, 512, 0, st>>>(W, scale, x, y, B, N, K, S); break;
        case 4: gemv_mfma_kernel<WT, 4, 4, EPI><<<grid, 256, 0, st>>>(W, scale, x, y, B, N, K, S); break;
        case 2: gemv_mfma_kernel<WT, 2, 4, EPI><<<grid, 128, 0, st>>>(W, scale, x, y, B, N, K, S); break;
        default: gemv_mfma_kernel<WT, 1, 4, EPI><<<grid, 64, 0, st>>>(W, scale, x, y, B, N, K, S); break;
    }
}

// y: [B, Nout] (Nout = S for SwiGLU). Batches above 16 run as consecutive chunks of at most 16 rows.
template <typename WT, int EPI>
int gemv_run(const char *name, const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int B, int Nout,
             int K, int rows, hipStream_t st) {
    LFM2Q_REQUIRE(W && x && y, LFM2Q_ERR_ARG, "%s: null pointer", name);
    LFM2Q_REQUIRE(sizeof(WT) == 2 || scale, LFM2Q_ERR_ARG, "%s: int8 W needs fp32 scale", name);
    LFM2Q_REQUIRE(B >= 1 && Nout >= 1 && K >= 64, LFM2Q_ERR_SHAPE, "%s: x [B, K], y [B, N] (B=%d N=%d K=%d)", name,
                  B, Nout, K);
    LFM2Q_REQUIRE(K % 64 == 0, LFM2Q_ERR_SHAPE, "%s: K must be a multiple of 64 (K=%d)", name, K);
    LFM2Q_REQUIRE(aligned16(W) && aligned16(x), LFM2Q_ERR_ALIGN, "%s: W and x must be 16-byte aligned", name);
    const int S = Nout;  // SwiGLU: w3 rows start at S
    for (int b0 = 0; b0 < B; b0 += 16) {
        const int bs = B - b0 < 16 ? B - b0 : 16;
        const uint16_t *xb = x + (size_t)b0 * K;
        uint16_t *yb = y + (size_t)b0 * Nout;
        if (bs == 1)
            launch_b1<WT, EPI>(W, scale, xb, yb, Nout, K, S, rows, st);
        else
            launch_mfma<WT, EPI>(W, scale, xb, yb, bs, Nout, K, S, st);
    }
    return launch_status(name);
}

}  // namespace
}  // namespace lfm2q

using namespace lfm2q;

extern "C" int lfm2q_gemv_w8(const int8_t *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *y, int B, int N,
                             int K, int rows, lfm2q_stream_t stream) {
    return gemv_run<int8_t, EPI_NONE>("gemv", W, scale, x, y, B, N, K, rows, (hipStream_t)stream);
}

extern "C" int lfm2q_gemv_bf16(const lfm2q_bf16 *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *y, int B,
                               int N, int K, int rows, lfm2q_stream_t stream) {
    return gemv_run<uint16_t, EPI_NONE>("gemv", W, scale, x, y, B, N, K, rows, (hipStream_t)stream);
}

extern "C" int lfm2q_gemv_swiglu(int wtype, const void *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *y,
                                 int B, int S, int K, lfm2q_stream_t stream) {
    if (wtype == 0)
        return gemv_run<int8_t, EPI_SWIGLU>("gemv_swiglu", (const int8_t *)W, scale, x, y, B, S, K, 0,
                                            (hipStream_t)stream);
    if (wtype == 1)
        return gemv_run<uint16_t, EPI_SWIGLU>("gemv_swiglu", (const uint16_t *)W, scale, x, y, B, S, K, 0,
                                              (hipStream_t)stream);
    return set_error(LFM2Q_ERR_ARG, "gemv_swiglu: wtype must be 0 (int8) or 1 (bf16), got %d", wtype);
}

extern "C" int lfm2q_gemv_residual(int wtype, const void *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *h,
                                   int B, int N, int K, lfm2q_stream_t stream) {
    if (wtype == 0)
        return gemv_run<int8_t, EPI_RESIDUAL>("gemv_residual", (const int8_t *)W, scale, x, h, B, N, K, 0,
                                              (hipStream_t)stream);
    if (wtype == 1)
        return gemv_run<uint16_t, EPI_RESIDUAL>("gemv_residual", (const uint16_t *)W, scale, x, h, B, N, K, 0,
                                                (hipStream_t)stream);
    return set_error(LFM2Q_ERR_ARG, "gemv_residual: wtype must be 0 (int8) or 1 (bf16), got %d", wtype);
}

extern "C" int lfm2q_silu_mul(const lfm2q_bf16 *g, lfm2q_bf16 *y, int B, int I, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(g && y, LFM2Q_ERR_ARG, "silu_mul: null pointer");
    LFM2Q_REQUIRE(B >= 1 && I >= 1 && B <= 65535, LFM2Q_ERR_SHAPE, "silu_mul: g [B, 2I], y [B, I] (B=%d I=%d)", B, I);
    silu_mul_kernel<<<dim3((I + 255) / 256, B), 256, 0, (hipStream_t)stream>>>(g, y, I);
    return launch_status("silu_mul");
}
