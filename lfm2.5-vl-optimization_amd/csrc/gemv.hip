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

#include <algorithm>

namespace lfm2q {
namespace {

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

__device__ __forceinline__ float apply_scale(float a, const float *__restrict__ scale, int n) {
    return scale ? a * scale[n] : a;
}

// ------------------------------------------------------------------------------------------------ batch 1
// Persistent batch-1 GEMV: about WPC wavefronts per CU, wavefront g handles output rows g, g + nw, g + 2 nw, ...
// (nw = wavefronts in the grid). K = 64 PER CPL: lane l owns the 16-byte chunks l, l + 64, ..., of every row, and
// its activations for those chunks stay in registers (packed bf16) for the whole kernel. The next row's weights are
// in flight while the current row is reduced (two register buffers used in turn), so every wavefront keeps its
// loads streaming instead of paying one memory latency per row. EPI_SWIGLU: a work item is the row pair (n, S + n).
template <typename WT, int CPL, int EPI>
__global__ __launch_bounds__(256) void gemv_b1p_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                       const uint16_t *__restrict__ x, uint16_t *__restrict__ y, int N,
                                                       int K, int S) {
    using D = PairDot<WT>;
    constexpr int PER = D::PER, XL = D::XL;
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int NB = CPL * NROW <= 2 ? 4 : 2;  // row buffers in the prefetch ring
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * 4;
    // row indices are wavefront-uniform: scale[] then goes through scalar loads, which do not wait on the vector
    // memory counter that tracks the next row's weights
    int n = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (n >= N) return;  // no block-level synchronization in this kernel
    v4i xr[CPL][XL];
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
        for (int q = 0; q < XL; ++q) xr[u][q] = ld16(x + (size_t)(lane + 64 * u) * PER + 8 * q);
    // one buffer resource per row (scalar base = the row, range = its K weights); each lane adds its fixed byte
    // offset, so no vector address arithmetic sits between a row's loads and the next row's
    const char *wbase = reinterpret_cast<const char *>(W);
    const uint32_t loff = lane * 16;
    const uint32_t rowb = (uint32_t)K * sizeof(WT);
    struct Item {
        v4i w[CPL][NROW];
        uint32_t h;  // EPI_RESIDUAL: the residual value, read together with the row's weights
    };
    auto load = [&](Item &it, int row) {
#pragma unroll
        for (int i = 0; i < NROW; ++i) {
            // rows past the end get an empty range: their loads return zeros without a memory access
            const rsrc_t rr = make_rsrc(wbase + (size_t)(i ? S + row : row) * rowb, row < N ? rowb : 0u);
#pragma unroll
            for (int u = 0; u < CPL; ++u) it.w[u][i] = buf_ld16_nt(rr, loff + u * 1024);
        }
        if (EPI == EPI_RESIDUAL) it.h = y[min(row, N - 1)];
    };
    auto finish = [&](const Item &it, int row) {
        float acc[NROW];
#pragma unroll
        for (int i = 0; i < NROW; ++i) {
            acc[i] = 0.f;
#pragma unroll
            for (int u = 0; u < CPL; ++u) acc[i] = D::dot(it.w[u][i], xr[u], acc[i]);
            acc[i] = wave_sum(acc[i]);
        }
        float v;
        if (EPI == EPI_NONE) {
            v = apply_scale(acc[0], scale, row);
        } else if (EPI == EPI_RESIDUAL) {
            v = bf2f(it.h) + rbf(apply_scale(acc[0], scale, row));
        } else {
            const float g = rbf(apply_scale(acc[0], scale, row));
            const float u = rbf(apply_scale(acc[NROW - 1], scale, S + row));
            v = rbf(silu_f32(g)) * u;
        }
        if (lane == 0) y[row] = (uint16_t)f2bf(v);
    };
    // NB row buffers used in turn: while a row is reduced, the NB - 1 rows after it are in flight (about 4-6 KiB
    // per wavefront, 32-48 KiB per CU at 8 wavefronts per CU: enough to cover the loaded HBM latency). Prefetches
    // are unconditional -- past the last row they go through an empty buffer range and cost no memory traffic --
    // because a conditional load would make the compiler wait for every outstanding load before the current row's
    // math, prefetches included.
    Item buf[NB];
#pragma unroll
    for (int j = 0; j < NB - 1; ++j) load(buf[j], n + j * nw);
    bool more = true;
    while (more) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (more) {
                load(buf[(j + NB - 1) % NB], n + (NB - 1) * nw);
                __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the current row's math
                finish(buf[j], n);
                n += nw;
                more = n < N;
            }
        }
    }
}

// One-shot batch-1 GEMV: one wavefront per R output rows, every wavefront exits after its rows (many wavefronts per
// CU in flight at once -- the better shape while a matrix is too small to give each of ~8 wavefronts per CU several
// rows). CPL > 0: K = 64 PER CPL, all of a wavefront's weight and activation loads are issued before the first
// dot. CPL == 0: any K % PER == 0, chunks streamed 8 per lane at a time. Per row, the arithmetic is that of the
// persistent kernel (same chunk order, same PairDot, same reduction), so either kernel gives the same bits.
template <typename WT, int R, int CPL, int EPI>
__global__ __launch_bounds__(256) void gemv_b1_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                      const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                      int N, int K, int S) {
    using D = PairDot<WT>;
    constexpr int PER = D::PER, XL = D::XL;
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 * R : R;
    const int lane = threadIdx.x & 63;
    const int n0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (threadIdx.x >> 6)) * R);
    if (n0 >= N) return;  // no block-level synchronization in this kernel
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

    if constexpr (CPL > 0) {
        v4i w[CPL][NROW], xr[CPL][XL];
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int i = 0; i < NROW; ++i) w[u][i] = ld_nt16(rp[i] + (size_t)(lane + 64 * u) * 16);
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int q = 0; q < XL; ++q) xr[u][q] = ld16(x + (size_t)(lane + 64 * u) * PER + 8 * q);
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int i = 0; i < NROW; ++i) acc[i] = D::dot(w[u][i], xr[u], acc[i]);
    } else {
        constexpr int U = 8;
        const int C = K / PER;
        for (int c0 = lane; c0 < C; c0 += 64 * U) {
            v4i w[U][NROW], xr[U][XL];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 64 * u;
#pragma unroll
                for (int i = 0; i < NROW; ++i) w[u][i] = c < C ? ld_nt16(rp[i] + (size_t)c * 16) : v4i{0, 0, 0, 0};
#pragma unroll
                for (int q = 0; q < XL; ++q) xr[u][q] = c < C ? ld16(x + (size_t)c * PER + 8 * q) : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (c0 + 64 * u < C)
#pragma unroll
                    for (int i = 0; i < NROW; ++i) acc[i] = D::dot(w[u][i], xr[u], acc[i]);
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
__device__ __forceinline__ v8bf i8x8_to_bf16(int d0, int d1) {
    v4u r;
    r[0] = pack_hi16((float)(int8_t)d0, (float)(int8_t)(d0 >> 8));
    r[1] = pack_hi16((float)(int8_t)(d0 >> 16), (float)(d0 >> 24));
    r[2] = pack_hi16((float)(int8_t)d1, (float)(int8_t)(d1 >> 8));
    r[3] = pack_hi16((float)(int8_t)(d1 >> 16), (float)(d1 >> 24));
    return __builtin_bit_cast(v8bf, r);
}
__device__ __forceinline__ v8bf as_bf16x8(v4i v) { return __builtin_bit_cast(v8bf, v); }

// WG = NWK wavefronts and 16 RT output rows (EPI_SWIGLU: plus the matching 16 RT rows of w3, so NT = 2 RT weight
// tiles). Wavefront w covers k in [w K/NWK, (w+1) K/NWK) in stages of U 64-k steps; all loads of a stage are
// issued before its MFMAs. In a step, lane (col = l%16, kq = l/16) loads k0 + 16 kq .. +15 of weight row
// (tile row) + col for every tile and of activation row col (if col < B): the activation loads are shared by the
// NT tiles, so the L2 traffic for x is B/(8 RT) of the weight bytes.
// MFMA layout (v_mfma_f32_16x16x32_bf16): A[i][k] from lane i + 16 (k/8), B[k][j] from lane j + 16 (k/8),
// D[i][j] in lane j + 16 (i/4), element i%4. A and B use the same k <-> (lane group, slot) map, so the product
// pairs x[m][k] with W[n][k] whatever order the hardware sums the 32 k in.
// The NWK partial tiles are summed in LDS in wavefront order, one tile at a time.
template <typename WT, int RT, int NWK, int U, int EPI>
__global__ __launch_bounds__(64 * NWK) void gemv_mfma_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                             const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                             int B, int N, int K, int S) {
    constexpr int NT = (EPI == EPI_SWIGLU ? 2 : 1) * RT;
    constexpr int WL = sizeof(WT) == 1 ? 1 : 2;  // 16-byte weight loads per lane per step
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 15, kq = lane >> 4;
    const int nbase = blockIdx.x * 16 * RT;
    const WT *wp[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int nl = min(nbase + 16 * (t % RT) + col, N - 1);
        wp[t] = W + (size_t)((EPI == EPI_SWIGLU && t >= RT ? S : 0) + nl) * K;
    }
    const bool xm = col < B;
    const uint16_t *xp = x + (size_t)(xm ? col : 0) * K;
    const int ks = K / NWK, kb = wave * ks, ke = kb + ks;

    v4f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int s0 = kb; s0 < ke; s0 += 64 * U) {
        v4i wv[U][NT][WL], xv[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = s0 + 64 * u + 16 * kq;
            const bool in = s0 + 64 * u < ke;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int h = 0; h < WL; ++h) wv[u][t][h] = in ? ld_nt16(wp[t] + k + 8 * h) : v4i{0, 0, 0, 0};
            xv[u][0] = (in && xm) ? ld16(xp + k) : v4i{0, 0, 0, 0};
            xv[u][1] = (in && xm) ? ld16(xp + k + 8) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + 64 * u < ke) {
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

    if constexpr (NWK > 1) {
        __shared__ v4f red[NWK][64];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t > 0) __syncthreads();  // wavefront 0 has read the previous tile
            red[wave][lane] = acc[t];
            __syncthreads();
            if (wave == 0) {
                v4f s = red[0][lane];
#pragma unroll
                for (int w = 1; w < NWK; ++w) s += red[w][lane];
                acc[t] = s;
            }
        }
        if (wave != 0) return;
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int n = nbase + 16 * t + col;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * kq + i;
            if (m >= B) continue;
            const float a = acc[t][i];
            if (EPI == EPI_NONE) {
                y[(size_t)m * N + n] = (uint16_t)f2bf(apply_scale(a, scale, n));
            } else if (EPI == EPI_RESIDUAL) {
                uint16_t *h = y + (size_t)m * N + n;
                *h = (uint16_t)f2bf(bf2f(*h) + rbf(apply_scale(a, scale, n)));
            } else {
                const float g = rbf(apply_scale(a, scale, n)), u = rbf(apply_scale(acc[RT + t][i], scale, S + n));
                y[(size_t)m * N + n] = (uint16_t)f2bf(rbf(silu_f32(g)) * u);
            }
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
// Batch 1. Persistent kernel (LFM2Q_GEMV_WPC wavefronts per CU, default 8: the read-stream optimum measured on
// MI355X) once every wavefront gets at least 8 rows, one-shot kernel (one wavefront per row) below that. Both need
// K = 64 PER CPL with CPL in {1, 2, 4, 8}; other K take the one-shot kernel's generic loop, where `rows` (1, 2, 4)
// sets the output rows per wavefront. Per-row arithmetic is the same in all of them.
template <typename WT, int EPI>
void launch_b1(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int N, int K, int S, int rows,
               hipStream_t st) {
    constexpr int PER = PairDot<WT>::PER;
    static const int wpc = env_int("LFM2Q_GEMV_WPC", 8);
    const int C = K / PER;
    const int cpl = C % 64 == 0 ? C / 64 : 0;
    const int blocks_p = device_cus() * (wpc < 4 ? 1 : wpc / 4);
    const bool persistent = (long)N >= 8L * 4 * blocks_p;
    const dim3 grid1((N + 3) / 4), gridp(std::min((N + 3) / 4, blocks_p));
#define LFM2Q_B1(C_)                                                                            \
    do {                                                                                        \
        if (persistent)                                                                         \
            gemv_b1p_kernel<WT, C_, EPI><<<gridp, 256, 0, st>>>(W, scale, x, y, N, K, S);       \
        else                                                                                    \
            gemv_b1_kernel<WT, 1, C_, EPI><<<grid1, 256, 0, st>>>(W, scale, x, y, N, K, S);     \
    } while (0)
    switch (cpl) {
        case 1: LFM2Q_B1(1); break;
        case 2: LFM2Q_B1(2); break;
        case 4: LFM2Q_B1(4); break;
        case 8: LFM2Q_B1(8); break;
        default: {
            auto grid = [&](int R) { return dim3((N + 4 * R - 1) / (4 * R)); };
            if (EPI == EPI_SWIGLU || rows <= 1)
                gemv_b1_kernel<WT, 1, 0, EPI><<<grid(1), 256, 0, st>>>(W, scale, x, y, N, K, S);
            else if (rows == 2)
                gemv_b1_kernel<WT, 2, 0, EPI><<<grid(2), 256, 0, st>>>(W, scale, x, y, N, K, S);
            else
                gemv_b1_kernel<WT, 4, 0, EPI><<<grid(4), 256, 0, st>>>(W, scale, x, y, N, K, S);
        }
    }
#undef LFM2Q_B1
}

// K split over NWK wavefronts, from K only (a plain and a fused call of the same weights then split alike, which
// keeps the fused epilogues bit-identical): 64-k steps per wavefront = U = 4 or 8, so one stage of loads holds all of
// a wavefront's work. Other K: the largest NWK <= 8 that divides the steps with at least 4 per wavefront, U = 4.
// RT (16-row tiles per wavefront): 4 for outputs of 32768+ rows, 2 from 8192 (or a SwiGLU pair from 4096 outputs),
// else 1 -- more tiles share each activation load, fewer workgroups remain for narrow outputs.
template <typename WT, int EPI>
void launch_mfma(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int B, int N, int K, int S,
                 hipStream_t st) {
    const int wide = EPI == EPI_SWIGLU ? 2 * N : N;
    const int rt = (wide >= 32768 && EPI != EPI_SWIGLU) ? 4 : (wide >= 8192 ? 2 : 1);
    const int steps = K / 64;
    auto grid = [&](int RT) { return dim3((N + 16 * RT - 1) / (16 * RT)); };
    if (steps == 128) {  // K = 8192: 16 wavefronts x 8 steps
        gemv_mfma_kernel<WT, 1, 16, 8, EPI><<<grid(1), 1024, 0, st>>>(W, scale, x, y, B, N, K, S);
    } else if (steps == 32) {  // K = 2048: 8 wavefronts x 4 steps
        if (rt == 4)
            gemv_mfma_kernel<WT, 4, 8, 4, EPI><<<grid(4), 512, 0, st>>>(W, scale, x, y, B, N, K, S);
        else if (rt == 2)
            gemv_mfma_kernel<WT, 2, 8, 4, EPI><<<grid(2), 512, 0, st>>>(W, scale, x, y, B, N, K, S);
        else
            gemv_mfma_kernel<WT, 1, 8, 4, EPI><<<grid(1), 512, 0, st>>>(W, scale, x, y, B, N, K, S);
    } else {
        int nwk = 1;
        for (int c = 8; c > 1; c >>= 1)
            if (steps % c == 0 && steps / c >= 4) {
                nwk = c;
                break;
            }
        switch (nwk) {
            case 8: gemv_mfma_kernel<WT, 1, 8, 4, EPI><<<grid(1), 512, 0, st>>>(W, scale, x, y, B, N, K, S); break;
            case 4: gemv_mfma_kernel<WT, 1, 4, 4, EPI><<<grid(1), 256, 0, st>>>(W, scale, x, y, B, N, K, S); break;
            case 2: gemv_mfma_kernel<WT, 1, 2, 4, EPI><<<grid(1), 128, 0, st>>>(W, scale, x, y, B, N, K, S); break;
            default: gemv_mfma_kernel<WT, 1, 1, 4, EPI><<<grid(1), 64, 0, st>>>(W, scale, x, y, B, N, K, S); break;
        }
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
