// Decode GEMVs for gfx950: y[b, n] = (sum_k W[n, k] x[b, k]) * scale[n] with int8 (weight-only) or bf16 weights,
// bf16 activations, fp32 accumulation, and optional fused SwiGLU / residual-add epilogues.
//
// The kernels are pure HBM streams over W (every weight byte is read exactly once per call):
//   gemv_b1_kernel    batch 1. One wavefront owns R output rows; lane l streams the 16-byte chunks l, l+64, ...
//                     of each row with non-temporal loads (a wavefront load = 1 KiB contiguous of one row), all of
//                     a lane's chunks are in flight before the first FMA. int8 -> fp32 is one SDWA convert per
//                     weight; the row sums of a wavefront's rows are reduced together (fold_sum). No LDS.
//   gemv_b1p_kernel   batch 1 on very tall matrices (131072+ rows at the default 8 wavefronts per CU): a persistent
//                     grid walks the rows, each wavefront's next row in flight while the current one is reduced.
//   gemv_bn_kernel    batch 2 with rows of at most 128 chunks: the batch-1 kernel over both batch rows, each weight
//                     chunk converted once.
//   gemv_mfma_kernel  batch 2..64. A workgroup owns RT tiles of 16 output rows (8 when the K run is split in two
//                     inside the MFMA, batches <= 16) and BT batch tiles of 16 (8) rows that share every weight
//                     load; its NWK wavefronts split K into 128-k blocks. A tile block is read by two wave loads of
//                     8 whole 128-byte lines; the weights are converted exactly to bf16 in registers and feed
//                     v_mfma_f32_16x16x32_bf16 with the activations as the A operand (batch rows x 32 k) and the
//                     weights as B (32 k x output rows). The partial tiles meet in LDS. The matrix cores take the
//                     batch FMAs off the VALU (about 1.5 VALU ops per weight at any batch).
// The per-row accumulation order of each kernel does not depend on which epilogue runs or on how many rows a
// wavefront owns, so the fused epilogues are bit-identical to the plain GEMV followed by the separate op.
//
// Reference: kernels/lfm2_decode.cu:429-950 (gemv_direct_kernel :576-661, gemv_epi_kernel :724-805,
// gemv_dispatch :667-706), kernels/lfm2_decode.cu:954-963 (silu_mul), :108-113 (residual rounding).
#include "common.hpp"
#include "gemv_math.hpp"
#include "rmsnorm.hpp"
#include "status.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

namespace lfm2q {
namespace {

// ------------------------------------------------------------------------------------------------ batch 1
// A batch-1 kernel's activations: lane l holds the XL vectors of 8 bf16 that chunk l + 64 u (u < CPL) multiplies,
// i.e. vectors XL (l + 64 u) + q. NORM: x is the RMSNorm of the row h with weight nw, computed here exactly as
// add_rmsnorm_q computes it (rmsnorm.hpp), so the GEMV of the normalized row equals add_rmsnorm_q followed by the
// GEMV bit for bit: the sum of squares is taken in add_rmsnorm_q's order -- lane l sums vectors c 64 + l, c < CH =
// CPL XL -- by fetching those vectors from the lanes that hold them (for XL = 2 vector c 64 + l is register
// [c / 2][l % 2] of lane 32 (c % 2) + l / 2; for XL = 1 the two layouts coincide), then x = bf16(w bf16(h rs))
// elementwise in the kernel's own layout. Needs K = 64 PER CPL exactly (every vector in range).
template <int PER, int XL, int CPL, bool NORM>
struct XLoadB1 {
    v4i hv[CPL][XL], wv[CPL][XL];
    // NORM: the row and the norm weight, in flight before the caller issues its weight loads
    __device__ __forceinline__ void issue(const uint16_t *__restrict__ x, const uint16_t *__restrict__ nw, int lane) {
        if constexpr (NORM) {
#pragma unroll
            for (int u = 0; u < CPL; ++u)
#pragma unroll
                for (int q = 0; q < XL; ++q) {
                    hv[u][q] = ld16(x + (size_t)(lane + 64 * u) * PER + 8 * q);
                    wv[u][q] = ld16(nw + (size_t)(lane + 64 * u) * PER + 8 * q);
                }
        }
    }
    __device__ __forceinline__ void finish(const uint16_t *__restrict__ x, float eps, int K, int lane,
                                           v4i (&xr)[CPL][XL]) {
        if constexpr (!NORM) {
#pragma unroll
            for (int u = 0; u < CPL; ++u)
#pragma unroll
                for (int q = 0; q < XL; ++q) xr[u][q] = ld16(x + (size_t)(lane + 64 * u) * PER + 8 * q);
        } else {
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < CPL * XL; ++c) {
                if constexpr (XL == 1) {
                    ss = sumsq8(hv[c][0], ss);
                } else {
                    const int src = 32 * (c & 1) + (lane >> 1);
                    v4i g;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int a = __shfl(hv[c >> 1][0][j], src), b = __shfl(hv[c >> 1][1][j], src);
                        g[j] = (lane & 1) ? b : a;
                    }
                    ss = sumsq8(g, ss);
                }
            }
            const float rs = rms_scale(wave_sum(ss), K, eps);
#pragma unroll
            for (int u = 0; u < CPL; ++u)
#pragma unroll
                for (int q = 0; q < XL; ++q)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        xr[u][q][j] = (int)rms_apply2((uint32_t)wv[u][q][j], (uint32_t)hv[u][q][j], rs);
        }
    }
};

// Persistent batch-1 GEMV: about WPC wavefronts per CU, wavefront g handles output rows g, g + nw, g + 2 nw, ...
// (nw = wavefronts in the grid). K = 64 PER CPL: lane l owns the 16-byte chunks l, l + 64, ..., of every row, and
// its activations for those chunks stay in registers (packed bf16) for the whole kernel. The next row's weights are
// in flight while the current row is reduced (two register buffers used in turn), so every wavefront keeps its
// loads streaming instead of paying one memory latency per row. EPI_SWIGLU: a work item is the row pair (n, S + n).
template <typename WT, int CPL, int EPI, bool NORM = false>
__global__ __launch_bounds__(256) void gemv_b1p_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                       const uint16_t *__restrict__ x, uint16_t *__restrict__ y, int N,
                                                       int K, int S, const uint16_t *__restrict__ normw = nullptr,
                                                       float eps = 0.f) {
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
    {
        XLoadB1<PER, XL, CPL, NORM> xl;
        xl.issue(x, normw, lane);
        xl.finish(x, eps, K, lane, xr);
    }
    // one buffer resource per row (scalar base = the row, range = its K weights); each lane adds its fixed byte
    // offset, so no vector address arithmetic sits between a row's loads and the next row's
    const char *wbase = reinterpret_cast<const char *>(W);
    const uint32_t loff = lane * 16;
    const uint32_t rowb = (uint32_t)K * sizeof(WT);
    struct Item {
        v4i w[CPL][NROW];
        float s[NROW];  // the rows' scales and (EPI_RESIDUAL) residual value, read together with the weights
        uint32_t h;
    };
    auto load = [&](Item &it, int row) {
        const int rc = min(row, N - 1);
#pragma unroll
        for (int i = 0; i < NROW; ++i) {
            // rows past the end get an empty range: their loads return zeros without a memory access
            const rsrc_t rr = make_rsrc(wbase + (size_t)(i ? S + row : row) * rowb, row < N ? rowb : 0u);
#pragma unroll
            for (int u = 0; u < CPL; ++u) it.w[u][i] = buf_ld16_nt(rr, loff + u * 1024);
            it.s[i] = scale ? scale[i ? S + rc : rc] : 1.f;
        }
        if (EPI == EPI_RESIDUAL) it.h = y[rc];
    };
    // NB rows (items) per round: their NROW NB per-lane partials are reduced together (fold_sum), and the lane that
    // holds item j's sums applies its epilogue and stores it, so reduction and epilogue run once per round
    constexpr int V = NROW * NB;
    constexpr int LPV = 64 / V;
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
        const int row0 = n;
        float part[V];  // value i NB + j: weight row i (w1, w3) of item j
        float sc[V];
        uint32_t hres[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (more) {
                load(buf[(j + NB - 1) % NB], n + (NB - 1) * nw);
                __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the current row's math
#pragma unroll
                for (int i = 0; i < NROW; ++i) {
                    float a = 0.f;
#pragma unroll
                    for (int u = 0; u < CPL; ++u) a = D::dot(buf[j].w[u][i], xr[u], a);
                    part[i * NB + j] = a;
                    sc[i * NB + j] = buf[j].s[i];
                }
                hres[j] = EPI == EPI_RESIDUAL ? buf[j].h : 0u;
                n += nw;
                more = n < N;
            } else {
#pragma unroll
                for (int i = 0; i < NROW; ++i) part[i * NB + j] = 0.f, sc[i * NB + j] = 1.f;
                hres[j] = 0u;
            }
        }
        const float r = fold_sum<V>(part);  // value v in lanes v 64 / V ...
        // SwiGLU: the w3 sum of item j sits 32 lanes above its w1 sum
        const float ru = EPI == EPI_SWIGLU ? __uint_as_float(__builtin_amdgcn_permlane32_swap(
                                                 __float_as_uint(r), __float_as_uint(r), false, false)[1])
                                           : 0.f;
        const int j = lane / LPV, row = row0 + j * nw;
        if (lane % LPV == 0 && j < NB && row < N) {
            float sg = 1.f, su = 1.f;
            uint32_t h = 0u;
#pragma unroll
            for (int jj = 0; jj < NB; ++jj)
                if (jj == j) sg = sc[jj], su = sc[(NROW - 1) * NB + jj], h = hres[jj];
            float v;
            if (EPI == EPI_NONE) {
                v = scale ? r * sg : r;
            } else if (EPI == EPI_RESIDUAL) {
                v = bf2f(h) + rbf(scale ? r * sg : r);
            } else {
                const float g = rbf(scale ? r * sg : r), u = rbf(scale ? ru * su : ru);
                v = rbf(silu_f32(g)) * u;
            }
            y[row] = (uint16_t)f2bf(v);
        }
    }
}

// One-shot batch-1 GEMV: one wavefront per R output rows, every wavefront exits after its rows (many wavefronts per
// CU in flight at once -- the better shape while a matrix is too small to give each of ~8 wavefronts per CU several
// rows). CPL > 0: K = 64 PER CPL, all of a wavefront's weight and activation loads are issued before the first
// dot. CPL == 0: any K % PER == 0, chunks streamed 8 per lane at a time. Per row, the arithmetic is that of the
// persistent kernel (same chunk order, same PairDot, same fold_sum lane pairing), so either kernel gives the same
// bits. XS (CPL > 0, not NORM): the workgroup's four wavefronts load the activation row once between them into LDS
// and each lane reads its chunks' vectors from there (the same values, so the same bits), instead of every
// wavefront fetching the whole row through L2 -- with one row per wavefront at K = 8192 that is 16 KiB of
// activations beside 8 KiB of weights per wavefront.
template <typename WT, int R, int CPL, int EPI, bool NORM = false, bool XS = false>
__global__ __launch_bounds__(256) void gemv_b1_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                      const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                      int N, int K, int S,
                                                      const uint16_t *__restrict__ normw = nullptr, float eps = 0.f) {
    using D = PairDot<WT>;
    constexpr int PER = D::PER, XL = D::XL;
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 * R : R;
    static_assert(!NORM || CPL > 0, "the normalizing form needs K = 64 PER CPL");
    static_assert(!XS || (CPL > 0 && !NORM), "the shared-activation form needs K = 64 PER CPL");
    const int lane = threadIdx.x & 63;
    const int n0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (threadIdx.x >> 6)) * R);
    // XS: every wavefront takes part in the workgroup's activation load and barrier; a wavefront past the last row
    // reads row N - 1 (the row pointers clamp) and stores nothing
    if (!XS && n0 >= N) return;  // no block-level synchronization in this kernel
    const char *rp[NROW];
#pragma unroll
    for (int i = 0; i < NROW; ++i) {
        const int orow = min(n0 + (i % R), N - 1);
        const int wrow = (EPI == EPI_SWIGLU && i >= R) ? S + orow : orow;
        rp[i] = reinterpret_cast<const char *>(W + (size_t)wrow * K);
    }
    // the epilogue's operands for the row this lane will store (lane i 64 / NROW stores row n0 + i), read first
    constexpr int LPV = 64 / NROW;
    const int ns = min(n0 + min(lane / LPV, R - 1), N - 1);
    const float sg = scale ? scale[ns] : 1.f, su = (EPI == EPI_SWIGLU && scale) ? scale[S + ns] : 1.f;
    const uint32_t h0 = EPI == EPI_RESIDUAL ? y[ns] : 0u;
    float acc[NROW];
#pragma unroll
    for (int i = 0; i < NROW; ++i) acc[i] = 0.f;

    if constexpr (CPL > 0 && XS) {
        // the row is NV vectors of 8 bf16; lane l's chunk l + 64 u multiplies vectors XL (l + 64 u) + q
        constexpr int NV = 64 * CPL * XL, VPT = (NV + 255) / 256;
        __shared__ v4i xs[NV];
        v4i w[CPL][NROW], xv[VPT], xr[CPL][XL];
#pragma unroll
        for (int j = 0; j < VPT; ++j)
            if (NV % 256 == 0 || (int)threadIdx.x + 256 * j < NV) xv[j] = ld16(x + (size_t)(threadIdx.x + 256 * j) * 8);
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int i = 0; i < NROW; ++i) w[u][i] = ld_nt16(rp[i] + (size_t)(lane + 64 * u) * 16);
#pragma unroll
        for (int j = 0; j < VPT; ++j)
            if (NV % 256 == 0 || (int)threadIdx.x + 256 * j < NV) xs[threadIdx.x + 256 * j] = xv[j];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int q = 0; q < XL; ++q) xr[u][q] = xs[XL * (lane + 64 * u) + q];
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int i = 0; i < NROW; ++i) acc[i] = D::dot(w[u][i], xr[u], acc[i]);
    } else if constexpr (CPL > 0) {
        v4i w[CPL][NROW], xr[CPL][XL];
        XLoadB1<PER, XL, CPL, NORM> xl;
        xl.issue(x, normw, lane);
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int i = 0; i < NROW; ++i) w[u][i] = ld_nt16(rp[i] + (size_t)(lane + 64 * u) * 16);
        xl.finish(x, eps, K, lane, xr);
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
    // all NROW row sums in one transposed reduction: row i's sum lands in lanes i 64 / NROW ...; SwiGLU: the w3 sum of
    // output i sits 32 lanes above its w1 sum
    const float r = fold_sum<NROW>(acc);
    const float ru = EPI == EPI_SWIGLU ? __uint_as_float(__builtin_amdgcn_permlane32_swap(
                                             __float_as_uint(r), __float_as_uint(r), false, false)[1])
                                       : 0.f;
    const int n = n0 + lane / LPV;
    if (lane % LPV != 0 || lane / LPV >= R || n >= N) return;
    if (EPI == EPI_NONE) {
        y[n] = (uint16_t)f2bf(scale ? r * sg : r);
    } else if (EPI == EPI_RESIDUAL) {
        y[n] = (uint16_t)f2bf(bf2f(h0) + rbf(scale ? r * sg : r));
    } else {
        const float g = rbf(scale ? r * sg : r), u = rbf(scale ? ru * su : ru);
        y[n] = (uint16_t)f2bf(rbf(silu_f32(g)) * u);
    }
}

// ------------------------------------------------------------------------------------------------ batch 2, VALU
// The one-shot batch-1 kernel over NB batch rows at once: each weight chunk is converted once and dotted with the NB
// rows' activations (all loads in flight before the first dot). Per batch row the arithmetic is the batch-1
// kernel's (same chunk order, PairDot and fold_sum), so each row of the result is bit-identical to a batch-1 call.
// For short rows only (K = 64 PER CPL, CPL <= 2): the activations of NB rows live in registers.
template <typename WT, int R, int CPL, int EPI, int NB>
__global__ __launch_bounds__(256) void gemv_bn_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                      const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                      int N, int K, int S, int B) {
    using D = PairDot<WT>;
    constexpr int PER = D::PER, XL = D::XL;
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 * R : R;
    static_assert(CPL >= 1, "K = 64 PER CPL");
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
    constexpr int LPV = 64 / NROW;
    const int ns = min(n0 + min(lane / LPV, R - 1), N - 1);
    const float sg = scale ? scale[ns] : 1.f, su = (EPI == EPI_SWIGLU && scale) ? scale[S + ns] : 1.f;
    uint32_t h0[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) h0[b] = (EPI == EPI_RESIDUAL && b < B) ? y[(size_t)b * N + ns] : 0u;
    // batch rows past B read zeros through an empty range
    const rsrc_t xr = make_rsrc(x, (uint32_t)B * K * 2u);
    v4i w[CPL][NROW], xv[NB][CPL][XL];
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
        for (int i = 0; i < NROW; ++i) w[u][i] = ld_nt16(rp[i] + (size_t)(lane + 64 * u) * 16);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int q = 0; q < XL; ++q)
                xv[b][u][q] = buf_ld16(xr, (uint32_t)(((size_t)b * K + (size_t)(lane + 64 * u) * PER + 8 * q) * 2));
    float acc[NB][NROW];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < NROW; ++i) acc[b][i] = 0.f;
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
        for (int i = 0; i < NROW; ++i)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[b][i] = D::dot(w[u][i], xv[b][u], acc[b][i]);
    const int n = n0 + lane / LPV;
    const bool st = lane % LPV == 0 && lane / LPV < R && n < N;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float r = fold_sum<NROW>(acc[b]);
        const float ru = EPI == EPI_SWIGLU ? __uint_as_float(__builtin_amdgcn_permlane32_swap(
                                                 __float_as_uint(r), __float_as_uint(r), false, false)[1])
                                           : 0.f;
        if (!st || b >= B) continue;
        uint16_t *yp = y + (size_t)b * N + n;
        if (EPI == EPI_NONE) {
            *yp = (uint16_t)f2bf(scale ? r * sg : r);
        } else if (EPI == EPI_RESIDUAL) {
            *yp = (uint16_t)f2bf(bf2f(h0[b]) + rbf(scale ? r * sg : r));
        } else {
            const float g = rbf(scale ? r * sg : r), u = rbf(scale ? ru * su : ru);
            *yp = (uint16_t)f2bf(rbf(silu_f32(g)) * u);
        }
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

// A workgroup owns RT tiles of TR = 16 / KS output rows (EPI_SWIGLU: plus the matching rows of w3, so NT = 2 RT
// weight tiles); its NWK wavefronts split K into contiguous runs of 128-k blocks, KB blocks per stage (at most 8
// weight loads per lane), every load of a stage issued before its MFMAs. v_mfma_f32_16x16x32_bf16 computes
// D[i][c] += sum_k A[i][k] B[k][c] over 16 x 16 outputs; column c of B is weight row c % TR over part c / TR of the
// wavefront's K run (KS parts of P blocks), row i of A is batch row i % TR over part i / TR of the same run, so the
// KS diagonal blocks D[TR s + b][TR s + r] are partial sums of output (b, r) and the others are discarded. KS = 2
// (8-row tiles, batches up to 8) doubles the workgroups of a narrow matrix at the price of idle MFMA lanes.
// MFMA m (m = 0..3) of a block takes 8 consecutive k per lane (lane l = c + 16 g):
//   int8 weights: k = 32 g + 8 m + s. A tile block (16 columns x 128 bytes) is read by two wave loads of 8 whole
//                 128-byte lines each (load q: lane l reads row l % 8 [+ 8 q for KS = 1] of part q [KS = 2], bytes
//                 16 (l / 8)), so every load covers full cache lines; one DPP row rotation by 8 lanes and three
//                 selects per dword then give lane (c, g) bytes 32 g .. 32 g + 31 of its column, converted exactly
//                 to bf16.
//   bf16 weights: k = 32 m + 8 g + s. Lane (c, g) loads the 16-byte pieces at byte offsets 16 g + 64 m of its
//                 column's block (piece m feeds MFMA m as loaded).
// The activation operand A holds x[batch][the same 8 k] in lane i + 16 g: four loads of 64 contiguous bytes per
// row and block (batch rows >= B read zeros), for int8 weights rearranged by a permlane transpose. A[i][k] and
// B[k][c] follow the same k <-> (lane group, slot) map, so the product pairs x[b][k] with W[r][k] whatever order the
// hardware sums the 32 k in; D[i][c] lands in lane c + 16 (i / 4), element i % 4.
// Every load goes through a buffer resource: rows past N, batch rows past B and k past K (a trailing half block)
// read zeros without a memory access. The partial tiles (NWK wavefronts x KS parts) are summed in LDS in a fixed
// order, every thread of the workgroup taking some of the outputs.
template <typename WT, int KS, int RT, int NWK, int EPI, int BT>
__global__ __launch_bounds__(64 * NWK) void gemv_mfma_kernel(const WT *__restrict__ W, const float *__restrict__ scale,
                                                             const uint16_t *__restrict__ x, uint16_t *__restrict__ y,
                                                             int B, int N, int K, int S) {
    constexpr bool I8 = sizeof(WT) == 1;
    constexpr int TR = 16 / KS;             // weight rows per tile, batch rows per part of a batch tile
    constexpr int NT = (EPI == EPI_SWIGLU ? 2 : 1) * RT;
    constexpr int WL = I8 ? 2 : 4;          // 16-byte weight loads per lane per tile per block
    // blocks per stage: at least 8 weight loads per lane in flight with one batch tile; with several, their
    // activation loads are in flight too and the registers run out first
    constexpr int KB = BT == 1 ? (NT * WL >= 8 ? 1 : 8 / (NT * WL)) : (NT * WL >= 4 || BT >= 4 ? 1 : 2);
    constexpr uint32_t BB = 128 * sizeof(WT);  // bytes of one row's block
    constexpr uint32_t OOR = 0x40000000u;   // an offset past every range below: the load returns zeros
    // the k range is wavefront-uniform: block conditions and offsets stay scalar where the lane does not matter
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int c = lane & 15, g = lane >> 4;
    const int nbase = blockIdx.x * TR * RT;
    const uint32_t rowb = (uint32_t)K * sizeof(WT);
    rsrc_t wr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int r0 = nbase + TR * (t % RT);
        const int rows = __builtin_amdgcn_readfirstlane(max(0, min(TR, N - r0)));  // keep the resource scalar
        wr[t] = make_rsrc(W + (size_t)((EPI == EPI_SWIGLU && t >= RT ? S : 0) + min(r0, N - 1)) * K,
                          (uint32_t)rows * rowb);
    }
    const rsrc_t xr = make_rsrc(x, (uint32_t)B * K * 2u);
    const int c8 = lane >> 3;  // int8: the lane's 16-byte chunk of a 128-byte row block
    const uint32_t woff = I8 ? (lane & 7) * rowb + 16 * c8 : (c % TR) * rowb + 16 * g;
    const int cpart = c / TR;  // part of this lane's B column (bf16) and A row
    const uint32_t xoff = (uint32_t)(c % TR) * K * 2u + 16 * g;  // batch tile j adds j TR rows

    // this wavefront's blocks [kb0, kb1): part s is kb0 + s P .. kb0 + s P + P - 1
    const int nblk = (K + 127) / 128;
    const int per = (nblk + NWK - 1) / NWK;
    const int kb0 = wave * per, kb1 = min(nblk, kb0 + per);
    const int P = (per + KS - 1) / KS;

    // Output elements (tile t, batch tile j, batch row b of the tile, row r -> y[TR j + b][nbase + TR t + r]).
    // Through LDS (NWK > 1 or KS > 1): thread threadIdx.x + 64 NWK i takes element TE (BT t + j) + TR b + r;
    // otherwise each lane keeps the 4 RT BT elements its MFMA accumulators hold (r = c, b = 4 g + e).
    constexpr bool VIA_LDS = NWK > 1 || KS > 1;
    constexpr int TE = TR * TR;
    constexpr int EL = VIA_LDS ? (RT * BT * TE + 64 * NWK - 1) / (64 * NWK) : 4 * RT * BT;
    struct Coord {
        int t, j, b, r;
    };
    auto coord = [&](int i) -> Coord {
        if constexpr (VIA_LDS) {
            const int idx = (int)threadIdx.x + i * 64 * NWK;
            return {idx / (BT * TE), (idx / TE) % BT, (idx % TE) / TR, idx % TR};
        } else {
            return {i / (4 * BT), (i >> 2) % BT, 4 * g + (i & 3), c};
        }
    };
    // the epilogue's operands (scales, residual values) are read before the weight stream starts, so their
    // latency is not paid again after the last MFMA
    float sg[EL], su[EL];
    uint32_t hr[EL];
#pragma unroll
    for (int i = 0; i < EL; ++i) {
        const Coord e = coord(i);
        const int n = min(nbase + TR * e.t + e.r, N - 1);  // rows past N are never stored
        const int bb = TR * e.j + e.b;
        sg[i] = scale ? scale[n] : 1.f;
        su[i] = (EPI == EPI_SWIGLU && scale) ? scale[S + n] : 1.f;
        hr[i] = (EPI == EPI_RESIDUAL && e.t < RT && bb < B) ? y[(size_t)bb * N + n] : 0u;
    }

    v4f acc[NT][BT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < BT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int b0 = kb0; b0 < kb0 + P; b0 += KB) {
        v4i wv[KB][NT][WL], xv[KB][BT][4];
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int b = b0 + u;  // block of part 0; part s reads block b + s P
            const bool step = b < kb0 + P;
#pragma unroll
            for (int h = 0; h < WL; ++h) {
                uint32_t o;
                if constexpr (I8) {
                    const int bh = b + (KS == 2 ? h * P : 0);
                    const bool in = step && bh < kb1 && bh * 128 + 16 * c8 < K;
                    o = in ? (KS == 1 ? 8 * h * rowb : 0u) + bh * BB : OOR;
                } else {
                    const int bl = b + cpart * P;
                    const bool in = step && bl < kb1 && bl * 128 + 32 * h < K;
                    o = in ? 64 * h + bl * BB : OOR;
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) wv[u][t][h] = buf_ld16_nt(wr[t], woff + o);
            }
            // activations: load p reads bytes 64 p + 16 g of the row's block (64 contiguous bytes per row); bf16
            // weights consume load p as MFMA p's operand, int8 weights after the transpose below
            const int bx = b + cpart * P;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const bool in = step && bx < kb1 && bx * 128 + 32 * p < K;
#pragma unroll
                for (int j = 0; j < BT; ++j)
                    xv[u][j][p] = buf_ld16(xr, xoff + (in ? j * TR * K * 2u + bx * 256 + 64 * p : OOR));
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the stage is in flight before the first wait
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            if constexpr (I8) {
                // lane (i, g) register p holds 16-byte chunk 4 p + g of the row's block; MFMA m needs chunk 4 g + m
                // (k = 32 g + 8 m). A 4 x 4 transpose over (register, 16-lane row): swap the upper 32 lanes of
                // registers 0, 1 with the lower 32 lanes of 2, 3, then the odd rows of 0, 2 with the even rows of 1, 3.
#pragma unroll
                for (int j = 0; j < BT; ++j)
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const auto s02 = __builtin_amdgcn_permlane32_swap(xv[u][j][0][d], xv[u][j][2][d], false, false);
                        const auto s13 = __builtin_amdgcn_permlane32_swap(xv[u][j][1][d], xv[u][j][3][d], false, false);
                        const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
                        const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
                        xv[u][j][0][d] = s01[0];
                        xv[u][j][1][d] = s01[1];
                        xv[u][j][2][d] = s23[0];
                        xv[u][j][3][d] = s23[1];
                    }
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                v4i q[2];  // int8: lane (c, g)'s bytes 32 g .. 32 g + 15 and 32 g + 16 .. 32 g + 31 of its column
                if constexpr (I8) {
                    // lanes c < 8 hold their column's chunk 2 g from load 0, lanes c >= 8 chunk 2 g + 1 from load 1;
                    // the other chunk sits in lane l ^ 8 of the other load (DPP row_ror:8 swaps the row halves)
                    const bool lowc = (lane & 8) == 0;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int a0 = wv[u][t][0][d], a1 = wv[u][t][1][d];
                        const int recv = __builtin_amdgcn_update_dpp(0, lowc ? a1 : a0, 0x128, 0xf, 0xf, false);
                        q[0][d] = lowc ? a0 : recv;
                        q[1][d] = lowc ? recv : a1;
                    }
                }
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    v8bf wb;
                    if constexpr (I8)
                        wb = i8x8_to_bf16(q[m >> 1][2 * (m & 1)], q[m >> 1][2 * (m & 1) + 1]);
                    else
                        wb = as_bf16x8(wv[u][t][m]);
#pragma unroll
                    for (int j = 0; j < BT; ++j)
                        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xv[u][j][m]), wb, acc[t][j], 0,
                                                                            0, 0);
                }
            }
        }
    }

    auto store = [&](int i, float a, float u) {
        const Coord e = coord(i);
        const int n = nbase + TR * e.t + e.r, bb = TR * e.j + e.b;
        if (e.t >= RT || n >= N || bb >= B) return;
        const float av = scale ? a * sg[i] : a;
        uint16_t *yp = y + (size_t)bb * N + n;
        if (EPI == EPI_NONE) {
            *yp = (uint16_t)f2bf(av);
        } else if (EPI == EPI_RESIDUAL) {
            *yp = (uint16_t)f2bf(bf2f(hr[i]) + rbf(av));
        } else {
            const float gv = rbf(av), uv = rbf(scale ? u * su[i] : u);
            *yp = (uint16_t)f2bf(rbf(silu_f32(gv)) * uv);
        }
    };
    if constexpr (VIA_LDS) {
        // wavefront w's tile t, batch tile j: D[i][c] at 4 (c + 16 (i / 4)) + i % 4 (lane c + 16 (i / 4), element
        // i % 4)
        __shared__ __attribute__((aligned(16))) float red[NWK][NT][BT][256];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int j = 0; j < BT; ++j) *reinterpret_cast<v4f *>(&red[wave][t][j][4 * lane]) = acc[t][j];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < EL; ++i) {
            const Coord e = coord(i);
            if (e.t >= RT || nbase + TR * e.t + e.r >= N || TR * e.j + e.b >= B) continue;
            float a = 0.f, u = 0.f;  // summed over wavefronts, then parts, in that fixed order
#pragma unroll
            for (int w = 0; w < NWK; ++w)
#pragma unroll
                for (int s = 0; s < KS; ++s) {
                    const int ii = TR * s + e.b, cc = TR * s + e.r;
                    const int at = 4 * (cc + 16 * (ii >> 2)) + (ii & 3);
                    const float va = red[w][e.t][e.j][at];
                    const float vu = EPI == EPI_SWIGLU ? red[w][NT - RT + e.t][e.j][at] : 0.f;
                    a = (w == 0 && s == 0) ? va : a + va;
                    u = (w == 0 && s == 0) ? vu : u + vu;
                }
            store(i, a, u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < EL; ++i) {
            const int t = i / (4 * BT), j = (i >> 2) % BT;
            store(i, acc[t][j][i & 3], acc[NT - RT + t][j][i & 3]);
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
// Batch 1. Persistent kernel (knob LFM2Q_GEMV_WPC wavefronts per CU, default 8: the read-stream optimum measured on
// MI355X) once every wavefront gets at least 64 rows (the 65536-row lm_head is 2.2 us faster one-shot), one-shot
// kernel below that with R output rows per wavefront:
// R = 2 from 6144 weight rows (half the wavefronts, each with twice the loads in flight and one reduction for both
// rows) and for the residual GEMVs of K <= 2048, else 1; the LFM2Q_GEMV_R knob (1, 2 or 4) overrides it where the
// registers allow, LFM2Q_GEMV_XS (0 / 1) the activation staging. Both need
// K = 64 PER CPL with CPL in {1, 2, 4, 8}; other K take the one-shot kernel's generic loop, where `rows` (1, 2, 4)
// sets the output rows per wavefront. Per-row arithmetic is the same in all of them.
template <typename WT, int EPI, bool NORM = false>
void launch_b1(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int N, int K, int S, int rows,
               hipStream_t st, const uint16_t *nw = nullptr, float eps = 0.f) {
    constexpr int PER = PairDot<WT>::PER;
    const int wpc = knob_int(KNOB_GEMV_WPC, 8);
    const int C = K / PER;
    const int cpl = C % 64 == 0 ? C / 64 : 0;
    const int blocks_p = device_cus() * (wpc < 4 ? 1 : wpc / 4);
    bool persistent = (long)N >= 64L * 4 * blocks_p;
    if (const KnobVal f = knob(KNOB_GEMV_PERSIST); f.n) persistent = f.v[0] != 0 && cpl > 0;  // forced
    int r1 = (EPI == EPI_SWIGLU ? 2L * N : (long)N) >= 6144 ? 2 : 1;
    // the normalizing form reads the input row and its norm weight and normalizes them once per wavefront: on the
    // large GEMVs four rows per wavefront share that work (MI355X runtime decode step 0.708 -> 0.702 ms; four rows
    // for the plain GEMVs too measured 0.3245 -> 0.3387 ms on the GEMV-only step, so only here)
    if (NORM && r1 == 2) r1 = 4;
    // the activation row staged in LDS once per workgroup (XS) where a wavefront reads at most two weight rows,
    // i.e. as many activation bytes as weight bytes or more; with it the K = 2048 residual GEMVs take two rows per
    // wavefront (MI355X, per launch in a graph: o/out_proj 3.96 -> 3.79 us, in_proj 4.54 -> 4.45, w2 5.31 -> 5.10;
    // w1|w3 + SwiGLU, four weight rows per wavefront, 7.15 -> 7.26 with it, so not there)
    const int xs_forced = knob_int(KNOB_GEMV_XS, -1);
    if (!NORM && xs_forced < 0 && EPI == EPI_RESIDUAL && cpl > 0 && cpl <= 2) r1 = 2;
    if (const KnobVal f = knob(KNOB_GEMV_R); f.n) r1 = f.v[0];
    const bool xs = !NORM && (xs_forced >= 0 ? xs_forced == 1 : (EPI == EPI_SWIGLU ? 2 * r1 : r1) <= 2);
    auto grid = [&](int R) { return dim3((N + 4 * R - 1) / (4 * R)); };
    const dim3 gridp(std::min((N + 3) / 4, blocks_p));
#define LFM2Q_B1R(R_, C_)                                                                                      \
    do {                                                                                                       \
        if (xs)                                                                                                \
            gemv_b1_kernel<WT, R_, C_, EPI, false, !NORM><<<grid(R_), 256, 0, st>>>(W, scale, x, y, N, K, S);  \
        else                                                                                                   \
            gemv_b1_kernel<WT, R_, C_, EPI, NORM><<<grid(R_), 256, 0, st>>>(W, scale, x, y, N, K, S, nw, eps); \
    } while (0)
#define LFM2Q_B1(C_)                                                                                        \
    do {                                                                                                    \
        if (persistent)                                                                                     \
            gemv_b1p_kernel<WT, C_, EPI, NORM><<<gridp, 256, 0, st>>>(W, scale, x, y, N, K, S, nw, eps);    \
        else if (r1 == 4 && C_ <= 2)                                                                        \
            LFM2Q_B1R(C_ <= 2 ? 4 : 1, C_);                                                                 \
        else if (r1 == 2 && C_ <= 4)                                                                        \
            LFM2Q_B1R(C_ <= 4 ? 2 : 1, C_);                                                                 \
        else                                                                                                \
            LFM2Q_B1R(1, C_);                                                                               \
    } while (0)
    switch (cpl) {
        case 1: LFM2Q_B1(1); break;
        case 2: LFM2Q_B1(2); break;
        case 4: LFM2Q_B1(4); break;
        case 8: LFM2Q_B1(8); break;
        default: {
            if constexpr (!NORM) {  // the normalizing form's entry point admits only the four K above
                if (EPI == EPI_SWIGLU || rows <= 1)
                    gemv_b1_kernel<WT, 1, 0, EPI><<<grid(1), 256, 0, st>>>(W, scale, x, y, N, K, S);
                else if (rows == 2)
                    gemv_b1_kernel<WT, 2, 0, EPI><<<grid(2), 256, 0, st>>>(W, scale, x, y, N, K, S);
                else
                    gemv_b1_kernel<WT, 4, 0, EPI><<<grid(4), 256, 0, st>>>(W, scale, x, y, N, K, S);
            }
        }
    }
#undef LFM2Q_B1
#undef LFM2Q_B1R
}

// Batch 2 on the VALU kernel when a row is at most 128 chunks (K <= 2048 int8, 1024 bf16), R as for batch 1
// (measured on MI355X: 4 % off the batch-2 decode step; at batch 3-4 the matrix-core kernel is faster). Returns
// false where it does not apply. The LFM2Q_GEMV_VALU knob = 0 turns it off.
template <typename WT, int EPI>
bool launch_bn(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int B, int N, int K, int S,
               hipStream_t st) {
    constexpr int PER = PairDot<WT>::PER;
    if (B != 2 || K % (64 * PER) || K / (64 * PER) > 2) return false;
    if (knob_int(KNOB_GEMV_VALU, 1) == 0) return false;
    const int cpl = K / (64 * PER);
    const int r = (EPI == EPI_SWIGLU ? 2L * N : (long)N) >= 6144 ? 2 : 1;
    const dim3 grid((N + 4 * r - 1) / (4 * r));
#define LFM2Q_BN(R_, C_) gemv_bn_kernel<WT, R_, C_, EPI, 2><<<grid, 256, 0, st>>>(W, scale, x, y, N, K, S, B)
    if (r == 2) {
        if (cpl == 1) LFM2Q_BN(2, 1); else LFM2Q_BN(2, 2);
    } else {
        if (cpl == 1) LFM2Q_BN(1, 1); else LFM2Q_BN(1, 2);
    }
#undef LFM2Q_BN
    return true;
}

// Launch shape from (weight rows, K, B) only -- a plain and a fused call over the same weights (w1|w3 as one
// [2 S, K] matrix) then split K alike, which keeps the fused epilogues bit-identical:
//   BT (batch tiles per wavefront, sharing every weight load): 16-row batch tiles, BT = 1, 2 or 4 for up to 16, 32
//   or 64 batch rows;
//   KS = 2 (8-row tiles, 256+ workgroups instead of 128) for at most 2048 weight rows: batch tiles of 8 rows, BT = 1
//   up to batch 8 and 2 up to batch 16;
//   RT = 2 for 6144+ weight rows (two tiles share each activation load) unless KS = 2, RT = 4 for 32768+ rows
//   without SwiGLU (the lm_head);
//   NWK from the 128-k blocks per wavefront: 2 when RT = 2 or BT > 1, 4 when KS = RT = BT = 1, 8 BT when KS = 2 (at
//   least 4 wavefronts with two batch tiles); at most 16 / BT (LDS), 8 / BT for 32768+ rows with several batch
//   tiles. Measured on MI355X over the LFM2 decode shapes at batches 4 to 64.
// The LFM2Q_GEMV_MFMA knob = "KS,RT,NWK[,BT]" overrides the shape (the last bits of the sums change with it).
template <typename WT, int EPI, int KS, int RT, int BT>
void launch_mfma_shape(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int B, int N, int K, int S,
                       int nwk, hipStream_t st) {
    const dim3 grid((N + (16 / KS) * RT - 1) / ((16 / KS) * RT));
#define LFM2Q_MF(NWK_) \
    gemv_mfma_kernel<WT, KS, RT, NWK_, EPI, BT><<<grid, 64 * NWK_, 0, st>>>(W, scale, x, y, B, N, K, S)
    constexpr int NWK_MAX = 16 / BT;  // LDS: NWK NT BT KiB of partial tiles with NT <= 4
    if constexpr (NWK_MAX >= 16)
        if (nwk >= 16) {
            LFM2Q_MF(16);
            return;
        }
    if constexpr (NWK_MAX >= 8)
        if (nwk >= 8) {
            LFM2Q_MF(8);
            return;
        }
    if (nwk >= 4)
        LFM2Q_MF(4);
    else if (nwk >= 2)
        LFM2Q_MF(2);
    else
        LFM2Q_MF(1);
#undef LFM2Q_MF
}

struct MfmaShape {
    int ks, rt, nwk, bt;
};

// B <= 64 (B <= 16 at KS = 2)
inline MfmaShape mfma_shape(int epi, long wrows, int B, int K) {
    const int nblk = (K + 127) / 128;
    MfmaShape m;
    m.ks = (B <= 16 && wrows <= 2048) ? 2 : 1;
    m.bt = m.ks == 2 ? (B <= 8 ? 1 : 2) : (B <= 16 ? 1 : B <= 32 ? 2 : 4);
    m.rt = (m.ks == 1 && wrows >= 6144) ? 2 : 1;
    const bool head = wrows >= 32768;
    if (epi != EPI_SWIGLU && head) m.rt = 4;  // halves the activation reads per weight byte again
    const int bpw = m.ks == 2 ? 8 * m.bt : (m.rt >= 2 || m.bt > 1) ? 2 : 4;  // target blocks per wavefront
    m.nwk = 1;
    while (m.nwk < 16 && (nblk >= bpw * 2 * m.nwk || (m.ks == 2 && m.bt > 1 && m.nwk < 4))) m.nwk *= 2;
    m.nwk = std::min(m.nwk, (head && m.bt > 1 ? 8 : 16) / m.bt);
    if (const KnobVal f = knob(KNOB_GEMV_MFMA); f.n) {
        const int got = f.n, fk = f.v[0], fr = f.v[1], fn = f.v[2], fb = f.n >= 4 ? f.v[3] : 1;
        const bool bt_ok = (fb == 1 || fb == 2 || (fb == 4 && fk == 1)) && B <= (16 / fk) * fb;
        const bool rt_ok = fr == 1 || (fr == 2 && fk == 1) || (fr == 4 && fk == 1 && epi != EPI_SWIGLU);
        if (got >= 3 && (fk == 1 || (fk == 2 && fr == 1)) && bt_ok && rt_ok &&
            (fn == 1 || fn == 2 || fn == 4 || fn == 8 || fn == 16) && fn <= 16 / fb)
            m = MfmaShape{fk, fr, fn, fb};
    }
    return m;
}

template <typename WT, int EPI>
void launch_mfma(const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int B, int N, int K, int S,
                 hipStream_t st) {
    const MfmaShape m = mfma_shape(EPI, EPI == EPI_SWIGLU ? 2L * S : N, B, K);
    auto go = [&](auto ks, auto rt, auto bt) {
        launch_mfma_shape<WT, EPI, decltype(ks)::value, decltype(rt)::value, decltype(bt)::value>(W, scale, x, y, B,
                                                                                                   N, K, S, m.nwk, st);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    auto with_bt = [&](auto ks, auto rt) {
        if (m.bt == 4)
            go(ks, rt, I4{});
        else if (m.bt == 2)
            go(ks, rt, I2{});
        else
            go(ks, rt, I1{});
    };
    if (m.ks == 2) {
        if (m.bt == 2)
            go(I2{}, I1{}, I2{});
        else
            go(I2{}, I1{}, I1{});
    } else if (m.rt == 4) {
        if constexpr (EPI != EPI_SWIGLU) with_bt(I1{}, I4{});
    } else if (m.rt == 2) {
        with_bt(I1{}, I2{});
    } else {
        with_bt(I1{}, I1{});
    }
}

// y: [B, Nout] (Nout = S for SwiGLU). Batches run as consecutive chunks of at most 64 rows (16 when the activations
// of 64 rows reach 1 GiB, or with the LFM2Q_GEMV_CHUNK knob = 16); a chunk of one row takes the batch-1
// kernels.
template <typename WT, int EPI>
int gemv_run(const char *name, const WT *W, const float *scale, const uint16_t *x, uint16_t *y, int B, int Nout,
             int K, int rows, hipStream_t st) {
    LFM2Q_REQUIRE(W && x && y, LFM2Q_ERR_ARG, "%s: null pointer", name);
    LFM2Q_REQUIRE(sizeof(WT) == 2 || scale, LFM2Q_ERR_ARG, "%s: int8 W needs fp32 scale", name);
    LFM2Q_REQUIRE(B >= 1 && Nout >= 1 && K >= 64, LFM2Q_ERR_SHAPE, "%s: x [B, K], y [B, N] (B=%d N=%d K=%d)", name,
                  B, Nout, K);
    LFM2Q_REQUIRE(K % 64 == 0, LFM2Q_ERR_SHAPE, "%s: K must be a multiple of 64 (K=%d)", name, K);
    LFM2Q_REQUIRE(K <= (1 << 24), LFM2Q_ERR_SHAPE, "%s: K above 16777216 (K=%d)", name, K);
    LFM2Q_REQUIRE(aligned16(W) && aligned16(x), LFM2Q_ERR_ALIGN, "%s: W and x must be 16-byte aligned", name);
    const int S = Nout;  // SwiGLU: w3 rows start at S
    // the activation resource of a chunk must stay below the out-of-range offset (1 GiB) the kernel uses
    int chunk = 64L * K * 2 < (1L << 30) ? 64 : 16;
    if (knob_int(KNOB_GEMV_CHUNK, 0) == 16) chunk = 16;
    for (int b0 = 0; b0 < B; b0 += chunk) {
        const int bs = B - b0 < chunk ? B - b0 : chunk;
        const uint16_t *xb = x + (size_t)b0 * K;
        uint16_t *yb = y + (size_t)b0 * Nout;
        if (bs == 1)
            launch_b1<WT, EPI>(W, scale, xb, yb, Nout, K, S, rows, st);
        else if (!launch_bn<WT, EPI>(W, scale, xb, yb, bs, Nout, K, S, st))
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

extern "C" int lfm2q_gemv_rmsnorm(int wtype, int epi, const void *W, const float *scale, const lfm2q_bf16 *h,
                                  const lfm2q_bf16 *norm_w, float eps, lfm2q_bf16 *y, int N, int K,
                                  lfm2q_stream_t stream) {
    const char *name = "gemv_rmsnorm";
    LFM2Q_REQUIRE(W && h && norm_w && y, LFM2Q_ERR_ARG, "%s: null pointer", name);
    LFM2Q_REQUIRE(wtype == 0 || wtype == 1, LFM2Q_ERR_ARG, "%s: wtype must be 0 (int8) or 1 (bf16), got %d", name,
                  wtype);
    LFM2Q_REQUIRE(epi == EPI_NONE || epi == EPI_SWIGLU, LFM2Q_ERR_ARG, "%s: epi must be 0 (none) or 1 (swiglu), got %d",
                  name, epi);
    LFM2Q_REQUIRE(wtype == 1 || scale, LFM2Q_ERR_ARG, "%s: int8 W needs fp32 scale", name);
    const int per_chunk = wtype == 0 ? 1024 : 512;  // K of one 16-byte weight chunk per lane
    LFM2Q_REQUIRE(N >= 1 && (K == per_chunk || K == 2 * per_chunk || K == 4 * per_chunk || K == 8 * per_chunk),
                  LFM2Q_ERR_SHAPE, "%s: N >= 1 and K in {%d, %d, %d, %d} (N=%d K=%d)", name, per_chunk, 2 * per_chunk,
                  4 * per_chunk, 8 * per_chunk, N, K);
    LFM2Q_REQUIRE(aligned16(W) && aligned16(h) && aligned16(norm_w), LFM2Q_ERR_ALIGN,
                  "%s: W, h and norm_w must be 16-byte aligned", name);
    const hipStream_t st = (hipStream_t)stream;
    if (wtype == 0) {
        if (epi == EPI_SWIGLU)
            launch_b1<int8_t, EPI_SWIGLU, true>((const int8_t *)W, scale, h, y, N, K, N, 0, st, norm_w, eps);
        else
            launch_b1<int8_t, EPI_NONE, true>((const int8_t *)W, scale, h, y, N, K, N, 0, st, norm_w, eps);
    } else {
        if (epi == EPI_SWIGLU)
            launch_b1<uint16_t, EPI_SWIGLU, true>((const uint16_t *)W, scale, h, y, N, K, N, 0, st, norm_w, eps);
        else
            launch_b1<uint16_t, EPI_NONE, true>((const uint16_t *)W, scale, h, y, N, K, N, 0, st, norm_w, eps);
    }
    return launch_status(name);
}

extern "C" int lfm2q_silu_mul(const lfm2q_bf16 *g, lfm2q_bf16 *y, int B, int I, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(g && y, LFM2Q_ERR_ARG, "silu_mul: null pointer");
    LFM2Q_REQUIRE(B >= 1 && I >= 1 && B <= 65535, LFM2Q_ERR_SHAPE, "silu_mul: g [B, 2I], y [B, I] (B=%d I=%d)", B, I);
    silu_mul_kernel<<<dim3((I + 255) / 256, B), 256, 0, (hipStream_t)stream>>>(g, y, I);
    return launch_status("silu_mul");
}
