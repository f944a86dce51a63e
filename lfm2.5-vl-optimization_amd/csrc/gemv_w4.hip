// INT4 weight-only decode GEMVs for gfx950: y[b, n] = sum_k s[n, g(k)] (q[n, k] - z[n, g(k)]) x[b, k], fp32
// accumulation, bf16 out, with the SwiGLU / residual epilogues of the INT8 GEMVs.
//
// Two weight formats, one nibble order (nibble i of 32-bit word w of a row holds weight k = 8 w + i):
//   fmt 0, the reference's: Wq uint8 [N, K/2] (weight 2j in the low nibble of byte j, stored as q + 8), scales
//          fp32 [N, K/group], zero point 8 for every group;
//   fmt 1, GPTQ-style:      Wq int32 [N, K/8], scales fp16 [N, K/group], zero points int32 [N, ceil(G/8)]
//          (nibble j of word w = zero point of group 8 w + j).
//
// Dequantization costs one or two bit operations per weight pair: ((word >> 4p) & 0x000F000F) | 0x43004300 (a shift
// for p > 0 and one v_and_or_b32) is the bf16 pair
// (128 + q[p], 128 + q[p + 4]) exactly (bf16 holds every integer in [128, 256)). A chunk's sum is then
//     sum_k s (q_k - z) x_k = s (sum_k (128 + q_k) x_k - (128 + z) sum_k x_k),
// with the first sum from v_dot2_f32_bf16 (batch 1) or bf16 MFMAs (batch 2..16) and the activation sums computed
// once per call (batch 1: per lane, in registers; MFMA: one extra MFMA against a matrix of ones, shared by all of a
// wavefront's weight tiles). The activations are repacked once into the matching (x[p], x[p + 4]) pairs.
//
// Reference: kernels/lfm2_decode.cu:826-950 (gemv_w4_kernel, launch_gemv_w4), bound as gemv_w4 in
// kernels/lfm2_decode.cpp:86-98; formats src/lfm2opt/quant.py:21-47 and src/lfm2opt/gptq.py:164-169.
#include "common.hpp"
#include "status.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace lfm2q {
namespace {

enum Epi { EPI_NONE = 0, EPI_SWIGLU = 1, EPI_RESIDUAL = 2 };

// The nibble masks as opaque register values: with the constants hidden from the optimizer, (a & m) | o selects a
// single v_and_or_b32 (a VOP3 instruction takes no literal operand on gfx9, so with visible constants the compiler
// emits a literal AND and a literal OR instead).
struct NibbleMasks {
    uint32_t m, o;  // 0x000F000F (SGPR), 0x43004300 (VGPR)
    __device__ NibbleMasks() {
        asm("s_mov_b32 %0, 0x000F000F" : "=s"(m));
        asm("v_mov_b32 %0, 0x43004300" : "=v"(o));
    }
    // (128 + q[p], 128 + q[p + 4]) as a bf16 pair, p = 0..3, from one 8-weight word
    __device__ uint32_t pair(uint32_t w, int p) const { return ((p ? w >> (4 * p) : w) & m) | o; }
};

// (x[p], x[p + 4]) from 8 bf16 activations x0..x7 held as 4 dwords (x0 | x1 << 16, ...)
__device__ __forceinline__ uint32_t xpair(const v4i &d, int p) {
    const uint32_t lo = (uint32_t)d[p >> 1], hi = (uint32_t)d[2 + (p >> 1)];
    return __builtin_amdgcn_perm(hi, lo, (p & 1) ? 0x07060302u : 0x05040100u);
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2bf as_bf16x2(uint32_t v) { return __builtin_bit_cast(v2bf, v); }
__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// Group scale and zero point of weight row `row`, group g: scale_raw / zero_raw are the loaded words, decoded by
// scale_of / zero_of where they are used, so that a load issued ahead of time is not waited for at its issue point
template <int FMT>
struct W4Fmt;
template <>
struct W4Fmt<0> {
    __device__ static uint32_t scale_raw(const void *S, int row, int g, int G) {
        return reinterpret_cast<const uint32_t *>(S)[(size_t)row * G + g];
    }
    __device__ static float scale_of(uint32_t r) { return __uint_as_float(r); }
    __device__ static uint32_t zero_raw(const int32_t *, int, int, int) { return 0u; }
    __device__ static int zero_of(uint32_t, int) { return 8; }
};
template <>
struct W4Fmt<1> {
    __device__ static uint32_t scale_raw(const void *S, int row, int g, int G) {
        return reinterpret_cast<const uint16_t *>(S)[(size_t)row * G + g];
    }
    __device__ static float scale_of(uint32_t r) { return h2f(r); }
    __device__ static uint32_t zero_raw(const int32_t *Z, int row, int g, int G) {
        return (uint32_t)Z[(size_t)row * ((G + 7) >> 3) + (g >> 3)];
    }
    __device__ static int zero_of(uint32_t r, int g) { return (r >> (4 * (g & 7))) & 15; }
};

__device__ __forceinline__ float epi_value(int epi, float a, float b, uint32_t h) {
    if (epi == EPI_NONE) return a;
    if (epi == EPI_RESIDUAL) return bf2f(h) + rbf(a);
    return rbf(silu_f32(rbf(a))) * rbf(b);
}

// ------------------------------------------------------------------------------------------------ batch 1
// Persistent: about WPC wavefronts per CU, wavefront g handles output rows g, g + nw, ... Lane l owns the 16-byte
// chunks (32 weights) c = l + 64 u, u < CPL, of every row; their activations stay in registers as bf16 pairs, with
// their sums. Each chunk lies in one group (group % 32 == 0), so a lane's partial is
// sum_u s_u (dot_u - (128 + z_u) xs_u). The next NB - 1 rows' weights, scales and zero points are in flight while a
// row is reduced; rows past the end go through an empty buffer range (zeros, no memory traffic). Chunks past K
// (K < 2048 CPL) read zeros through the row's buffer range and have zero activations.
template <int FMT, int CPL, int EPI>
__global__ __launch_bounds__(256) void gemv_w4_b1_kernel(const uint8_t *__restrict__ Wq, const void *__restrict__ S,
                                                         const int32_t *__restrict__ Z, const uint16_t *__restrict__ x,
                                                         uint16_t *__restrict__ y, int N, int K, int group, int Sr) {
    using F = W4Fmt<FMT>;
    const NibbleMasks nm;
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int NB = CPL * NROW <= 2 ? 4 : 2;
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * 4;
    const int G = K / group;
    // A wavefront without rows (n >= N, the tail of the last workgroup) still takes its part of the shared activation
    // repack below, then runs one round of empty rows (zero-range loads, no stores).
    int n = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));

    int gl[CPL];  // group of the lane's chunk u (clamped for chunks past K)
#pragma unroll
    for (int u = 0; u < CPL; ++u) gl[u] = min(32 * (lane + 64 * u) / group, G - 1);
    const uint32_t rowb = (uint32_t)K / 2;
    struct Item {
        v4i w[CPL][NROW];
        uint32_t s[CPL][NROW], z[CPL][NROW];  // raw scale and zero-point words
        uint32_t h;
    };
    auto load = [&](Item &it, int row) {
        const int rc = min(row, N - 1);
#pragma unroll
        for (int i = 0; i < NROW; ++i) {
            const int wr = i ? Sr + row : row, wc = i ? Sr + rc : rc;
            const rsrc_t rr = make_rsrc(Wq + (size_t)wr * rowb, row < N ? rowb : 0u);
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                it.w[u][i] = buf_ld16_nt(rr, (lane + 64 * u) * 16);
                it.s[u][i] = F::scale_raw(S, wc, gl[u], G);
                it.z[u][i] = F::zero_raw(Z, wc, gl[u], G);
            }
        }
        if (EPI == EPI_RESIDUAL) it.h = y[rc];
    };
    // The activation pairs of chunk c = lane + 64 u are the same for every wavefront, so the workgroup converts them
    // once: wavefront j converts piece j (8 activations) of every chunk into LDS, then each lane reads its chunks'
    // 16 pairs and 4 piece sums back. xp[u][4 j + p] = (x[8 j + p], x[8 j + p + 4]), word-major. The activation
    // loads go first and the first rows' weights right after them, so the repack waits only for the activations
    // while the weights stay in flight.
    __shared__ uint32_t xq[CPL][16][64];
    __shared__ float xsq[CPL][4][64];
    const int jx = threadIdx.x >> 6;
    const rsrc_t xr = make_rsrc(x, (uint32_t)K * 2u);  // chunks past K read zeros (no branch around the loads)
    v4i xd[CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u) xd[u] = buf_ld16(xr, (uint32_t)(lane + 64 * u) * 64u + 16u * jx);
    Item buf[NB];
#pragma unroll
    for (int j = 0; j < NB - 1; ++j) load(buf[j], n + j * nw);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
#pragma unroll
        for (int p = 0; p < 4; ++p) xq[u][4 * jx + p][lane] = xpair(xd[u], p);
        float t = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) t += bf2f_lo((uint32_t)xd[u][e]) + bf2f_hi((uint32_t)xd[u][e]);
        xsq[u][jx][lane] = t;
    }
    // LDS writes done, then the workgroup barrier; a bare s_barrier, because __syncthreads()' fence would also wait
    // for the weight loads in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    uint32_t xp[CPL][16];
    float xs[CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
#pragma unroll
        for (int q = 0; q < 16; ++q) xp[u][q] = xq[u][q][lane];
        xs[u] = ((xsq[u][0][lane] + xsq[u][1][lane]) + xsq[u][2][lane]) + xsq[u][3][lane];
    }
    // a row's per-lane partial: sum_u s_u (dot_u - (128 + z_u) xs_u)
    auto partial = [&](const Item &it, int i) {
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int p = 0; p < 4; ++p)
                    d = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nm.pair((uint32_t)it.w[u][i][j], p)),
                                                        as_bf16x2(xp[u][4 * j + p]), d, false);
            acc += F::scale_of(it.s[u][i]) * (d - (float)(128 + F::zero_of(it.z[u][i], gl[u])) * xs[u]);
        }
        return acc;
    };
    // NB rows (items) per round; their NROW NB partials are reduced together (fold_sum) and the lane holding item
    // j's sum applies the epilogue and stores it, so the reduction and the epilogue run once per round
    constexpr int V = NROW * NB;
    bool more = true;
    while (more) {
        const int row0 = n;
        float part[V];  // value i NB + j: weight row i (w1, w3) of item j
        uint32_t hres[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (more) {
                load(buf[(j + NB - 1) % NB], n + (NB - 1) * nw);
                __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the current row's math
#pragma unroll
                for (int i = 0; i < NROW; ++i) part[i * NB + j] = partial(buf[j], i);
                hres[j] = EPI == EPI_RESIDUAL ? buf[j].h : 0u;
                n += nw;
                more = n < N;
            } else {
#pragma unroll
                for (int i = 0; i < NROW; ++i) part[i * NB + j] = 0.f;
                hres[j] = 0u;
            }
        }
        const float r = fold_sum<V>(part);  // value v in lanes v 64 / V ...
        // SwiGLU: the w3 sum of item j sits 32 lanes above its w1 sum
        const float u = EPI == EPI_SWIGLU ? __uint_as_float(__builtin_amdgcn_permlane32_swap(
                                                __float_as_uint(r), __float_as_uint(r), false, false)[1])
                                          : 0.f;
        constexpr int LPV = 64 / V;
        const int j = lane / LPV, row = row0 + j * nw;
        if (lane % LPV == 0 && j < NB && row < N) {
            uint32_t h = 0u;
#pragma unroll
            for (int jj = 0; jj < NB; ++jj)
                if (jj == j) h = hres[jj];
            y[row] = (uint16_t)f2bf(epi_value(EPI, r, u, h));
        }
    }
}

// One-shot batch 1: wavefront w of workgroup b owns output rows (4 b + w) R .. + R - 1, issues all their weight,
// scale and zero-point loads after its activation loads, and exits after them (many short wavefronts streaming
// through the CUs, so one's dequantization overlaps the loads of those dispatched after it; the persistent kernel
// issues every wavefront's rows up front and dequantizes them all at the end). Each wavefront converts its own
// chunks' activations in registers (no LDS, no barrier) with the persistent kernel's arithmetic, so each row's bits
// are the same as gemv_w4_b1_kernel's. Used below 32768 weight rows (measured: the decode step's w1|w3 6.5 -> 5.5
// us, in_proj 4.1 -> 3.8 us; the 65536-row lm_head stays faster persistent).
// XS: the workgroup repacks the activation row once between its four wavefronts -- thread t converts chunks t,
// t + 256, ... with the same arithmetic into LDS (pair vector j of chunk c at xpv[j][c], its activation sum at
// xsv[c]) -- and every lane reads its chunks' pairs from there, instead of every wavefront loading the whole row
// and repacking it (same values, so the same bits).
template <int FMT, int CPL, int EPI, int R, bool XS = false>
__global__ __launch_bounds__(256) void gemv_w4_b1o_kernel(const uint8_t *__restrict__ Wq, const void *__restrict__ S,
                                                          const int32_t *__restrict__ Z, const uint16_t *__restrict__ x,
                                                          uint16_t *__restrict__ y, int N, int K, int group, int Sr) {
    using F = W4Fmt<FMT>;
    const NibbleMasks nm;
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int V = NROW * R;
    constexpr int NC = 64 * CPL, CPT = XS ? (NC + 255) / 256 : CPL;  // chunks of a row; chunks loaded per thread
    const int lane = threadIdx.x & 63;
    const int n0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (threadIdx.x >> 6)) * R);
    // XS: every wavefront takes part in the workgroup's activation repack and barrier; one past the last row reads
    // row N - 1's scales (clamped) through an empty weight range and stores nothing
    if (!XS && n0 >= N) return;  // no block-level synchronization in this kernel
    const int G = K / group;
    int gl[CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u) gl[u] = min(32 * (lane + 64 * u) / group, G - 1);
    const uint32_t rowb = (uint32_t)K / 2;
    // activations first (cache hits), then every row's weights, scales and zero points; the activations of chunk c
    // are bytes 64 c .. 64 c + 63 of x (chunks past K read zeros through the range)
    const rsrc_t xr = make_rsrc(x, (uint32_t)K * 2u);
    v4i xd[CPT][4];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = XS ? (int)threadIdx.x + 256 * u : lane + 64 * u;
        if (!XS || NC % 256 == 0 || c < NC)
#pragma unroll
            for (int j = 0; j < 4; ++j) xd[u][j] = buf_ld16(xr, (uint32_t)c * 64u + 16u * j);
    }
    v4i w[R][NROW][CPL];
    uint32_t sr[R][NROW][CPL], zr[R][NROW][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < NROW; ++i) {
            const int row = n0 + r, rc = min(row, N - 1);
            const int wr = i ? Sr + row : row, wc = i ? Sr + rc : rc;
            const rsrc_t rr = make_rsrc(Wq + (size_t)wr * rowb, row < N ? rowb : 0u);
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                w[r][i][u] = buf_ld16_nt(rr, (lane + 64 * u) * 16);
                sr[r][i][u] = F::scale_raw(S, wc, gl[u], G);
                zr[r][i][u] = F::zero_raw(Z, wc, gl[u], G);
            }
        }
    const int ns = min(n0 + min(lane / (64 / V), R - 1), N - 1);
    const uint32_t h0 = EPI == EPI_RESIDUAL ? y[ns] : 0u;
    uint32_t xp[CPL][16];
    float xs[CPL];
    // chunk pairs (x[p], x[p + 4]) of each 8-value vector and the chunk's activation sum
    auto repack = [&](const v4i(&d)[4], uint32_t(&pp)[16], float &sum) {
        float t4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int p = 0; p < 4; ++p) pp[4 * j + p] = xpair(d[j], p);
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) t += bf2f_lo((uint32_t)d[j][e]) + bf2f_hi((uint32_t)d[j][e]);
            t4[j] = t;
        }
        sum = ((t4[0] + t4[1]) + t4[2]) + t4[3];
    };
    if constexpr (XS) {
        __shared__ v4i xpv[4][NC];
        __shared__ float xsv[NC];
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int c = (int)threadIdx.x + 256 * u;
            if (NC % 256 == 0 || c < NC) {
                uint32_t pp[16];
                float sum;
                repack(xd[u], pp, sum);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    xpv[j][c] = v4i{(int)pp[4 * j], (int)pp[4 * j + 1], (int)pp[4 * j + 2], (int)pp[4 * j + 3]};
                xsv[c] = sum;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v4i v = xpv[j][lane + 64 * u];
#pragma unroll
                for (int p = 0; p < 4; ++p) xp[u][4 * j + p] = (uint32_t)v[p];
            }
            xs[u] = xsv[lane + 64 * u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < CPL; ++u) repack(xd[u], xp[u], xs[u]);
    }
    float part[V];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < NROW; ++i) {
            float acc = 0.f;
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                float d = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        d = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nm.pair((uint32_t)w[r][i][u][j], p)),
                                                            as_bf16x2(xp[u][4 * j + p]), d, false);
                acc += F::scale_of(sr[r][i][u]) * (d - (float)(128 + F::zero_of(zr[r][i][u], gl[u])) * xs[u]);
            }
            part[i * R + r] = acc;
        }
    const float rs = fold_sum<V>(part);
    const float us = EPI == EPI_SWIGLU ? __uint_as_float(__builtin_amdgcn_permlane32_swap(
                                             __float_as_uint(rs), __float_as_uint(rs), false, false)[1])
                                       : 0.f;
    constexpr int LPV = 64 / V;
    const int r = lane / LPV, row = n0 + r;
    if (lane % LPV != 0 || r >= R || row >= N) return;
    y[row] = (uint16_t)f2bf(epi_value(EPI, rs, us, h0));
}

// ------------------------------------------------------------------------------------------------ batch 2..16
// A workgroup owns RT tiles of TR = 16 / KS output rows (EPI_SWIGLU: plus the matching w3 rows, NT = 2 RT tiles);
// its NWK wavefronts split K into contiguous runs of 256-k blocks (one 128-byte line per row), KB blocks per stage,
// every load of a stage issued before its MFMAs. v_mfma_f32_16x16x32_bf16 computes D[i][c] += sum_k A[i][k] B[k][c];
// column c of B is weight row c % TR over part c / TR of the wavefront's K run (KS parts of P blocks), row i of A is
// batch row i % TR over part i / TR, so the KS diagonal blocks D[TR s + b][TR s + r] are partial sums of output
// (b, r) and the others are discarded (KS = 2: 8-row tiles, batches up to 8, twice the workgroups).
// Weights: lane (c, g) (l = c + 16 g) needs 16-byte chunks g and g + 4 (k = 32 g and 128 + 32 g) of its column's
// block. Load q reads 8 whole lines -- rows c % 8 (+ 8 q for KS = 1) of part q (KS = 2) -- lane (c, g) taking chunk
// g + 4 ((c / 8) ^ q): each lane gets its chunk g from one load and its chunk g + 4 sits in lane l ^ 8 of the other
// (one DPP row rotation by 8 and three selects per dword). MFMA (h, j), h = chunk half, j = word: lane group g
// slot s holds k = 128 h + 32 g + 8 j + perm(s) with perm pairing nibbles (p, p + 4) -- the 32 k of one MFMA lie in
// one 128-k group, so the group's scale and zero point apply to its result: per tile and half,
//     acc += s (sum_j D_j - (128 + z) sum_j X_j),   X_j = the same MFMA against a matrix of ones.
// Activations: load p reads bytes 64 p + 16 g of the row's 512-byte block (64 contiguous bytes per row); two 4 x 4
// permlane transposes give lane (i, g) x[i][128 h + 32 g + 8 j .. + 7] in register 4 h + j.
// Every load goes through a buffer resource (rows past N, batch rows past B and k past K read zeros). The partial
// tiles (NWK wavefronts x KS parts) are summed in LDS in a fixed order, every thread taking some of the outputs.
template <int FMT, int KS, int RT, int NWK, int EPI>
__global__ __launch_bounds__(64 * NWK) void gemv_w4_mfma_kernel(const uint8_t *__restrict__ Wq,
                                                                const void *__restrict__ S,
                                                                const int32_t *__restrict__ Z,
                                                                const uint16_t *__restrict__ x,
                                                                uint16_t *__restrict__ y, int B, int N, int K,
                                                                int group, int Sr) {
    using F = W4Fmt<FMT>;
    const NibbleMasks nm;
    constexpr int TR = 16 / KS;
    constexpr int NT = (EPI == EPI_SWIGLU ? 2 : 1) * RT;
    constexpr int KB = 2;                   // blocks per stage (a block holds 8 activation registers per lane)
    constexpr uint32_t OOR = 0x40000000u;   // an offset past every range below: the load returns zeros
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int c = lane & 15, g = lane >> 4;
    const int nbase = blockIdx.x * TR * RT;
    const int G = K / group;
    const uint32_t rowb = (uint32_t)K / 2;
    rsrc_t wr[NT];
    int srow[NT];  // the weight row of this lane's column, for its scales and zero points
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int r0 = nbase + TR * (t % RT), off = EPI == EPI_SWIGLU && t >= RT ? Sr : 0;
        const int rows = __builtin_amdgcn_readfirstlane(max(0, min(TR, N - r0)));  // keep the resource scalar
        wr[t] = make_rsrc(Wq + (size_t)(off + min(r0, N - 1)) * rowb, (uint32_t)rows * rowb);
        srow[t] = off + min(r0 + c % TR, N - 1);
    }
    const rsrc_t xr = make_rsrc(x, (uint32_t)B * K * 2u);
    const int cpart = c / TR;  // part of this lane's B column and A row
    const uint32_t xoff = (uint32_t)(c % TR) * K * 2u + 16 * g;
    const v8bf ones = __builtin_bit_cast(v8bf, v4u{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

    const int nblk = (K + 255) / 256;
    const int per = (nblk + NWK - 1) / NWK;
    const int kb0 = wave * per, kb1 = min(nblk, kb0 + per);
    const int P = (per + KS - 1) / KS;

    // Output elements (tile t, batch row b, row r -> y[b][nbase + TR t + r]): thread threadIdx.x + 64 NWK i takes
    // element TR TR t + TR b + r of the summed tiles.
    constexpr int TE = TR * TR;
    constexpr int EL = (RT * TE + 64 * NWK - 1) / (64 * NWK);
    struct Coord {
        int t, b, r;
    };
    auto coord = [&](int i) -> Coord {
        const int idx = (int)threadIdx.x + i * 64 * NWK;
        return {idx / TE, (idx % TE) / TR, idx % TR};
    };
    // the residual values are read before the weight stream starts (their latency is not paid after the last MFMA)
    uint32_t hr[EL];
#pragma unroll
    for (int i = 0; i < EL; ++i) {
        const Coord e = coord(i);
        const int n = min(nbase + TR * e.t + e.r, N - 1);
        hr[i] = (EPI == EPI_RESIDUAL && e.t < RT && e.b < B) ? y[(size_t)e.b * N + n] : 0u;
    }

    v4f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int b0 = kb0; b0 < kb0 + P; b0 += KB) {
        v4i wv[KB][NT][2], xv[KB][8];
        // The stage's scales and zero points: 2 blocks x 2 halves = 4 groups per column. Lane (c, j) loads group
        // gi(u = j / 2, h = j % 2) of its column's row, one load per tile instead of one per (block, half); lane
        // (c, g) later takes group (u, h) from lane c + 16 (2 u + h). Raw words, decoded at their use.
        static_assert(KB == 2, "one lane group per (block, half) of the stage");
        uint32_t scr[NT], zpr[NT];
        {
            const int gj = min((min(b0 + (g >> 1) + cpart * P, nblk - 1) * 256 + 128 * (g & 1)) / group, G - 1);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                scr[t] = F::scale_raw(S, srow[t], gj, G);
                zpr[t] = F::zero_raw(Z, srow[t], gj, G);
            }
        }
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int b = b0 + u;  // block of part 0; part s reads block b + s P
            const bool step = b < kb0 + P;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int bq = b + (KS == 2 ? q * P : 0);
                const int ch = g + 4 * (((c >> 3) ^ q) & 1);
                const bool in = step && bq < kb1 && bq * 256 + 32 * ch < K;
                const uint32_t o = ((c & 7) + (KS == 1 ? 8 * q : 0)) * rowb + 16 * ch + bq * 128u;
#pragma unroll
                for (int t = 0; t < NT; ++t) wv[u][t][q] = buf_ld16_nt(wr[t], in ? o : OOR);
            }
            const int bx = b + cpart * P;
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const bool in = step && bx < kb1 && bx * 256 + 32 * p < K;
                xv[u][p] = buf_ld16(xr, xoff + (in ? bx * 512 + 64 * p : OOR));
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the stage is in flight before the first wait
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            // lane (i, g) register p holds 16-byte chunk 4 p + g; MFMA (h, j) needs chunk 16 h + 4 g + j, held by
            // lane j in register 4 h + g: two 4 x 4 transposes over (register, 16-lane row)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    v4i &r0 = xv[u][4 * h], &r1 = xv[u][4 * h + 1], &r2 = xv[u][4 * h + 2], &r3 = xv[u][4 * h + 3];
                    const auto s02 = __builtin_amdgcn_permlane32_swap(r0[d], r2[d], false, false);
                    const auto s13 = __builtin_amdgcn_permlane32_swap(r1[d], r3[d], false, false);
                    const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
                    const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
                    r0[d] = s01[0];
                    r1[d] = s01[1];
                    r2[d] = s23[0];
                    r3[d] = s23[1];
                }
            v8bf a[8];
            v4f dx[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                dx[h] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v4i &xr4 = xv[u][4 * h + j];
                    a[4 * h + j] = __builtin_bit_cast(v8bf, v4u{xpair(xr4, 0), xpair(xr4, 1), xpair(xr4, 2), xpair(xr4, 3)});
                    dx[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[4 * h + j], ones, dx[h], 0, 0, 0);
                }
            }
            const bool lowc = (lane & 8) == 0;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                v4i q2[2];  // chunk g and chunk g + 4 of this lane's column
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) {
                    const int a0 = wv[u][t][0][dd], a1 = wv[u][t][1][dd];
                    const int recv = __builtin_amdgcn_update_dpp(0, lowc ? a1 : a0, 0x128, 0xf, 0xf, false);
                    q2[0][dd] = lowc ? a0 : a1;
                    q2[1][dd] = recv;
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    v4f d = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t w = (uint32_t)q2[h][j];
                        const v8bf bw4 = __builtin_bit_cast(v8bf, v4u{nm.pair(w, 0), nm.pair(w, 1), nm.pair(w, 2), nm.pair(w, 3)});
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[4 * h + j], bw4, d, 0, 0, 0);
                    }
                    const int gi = min((min(b0 + u + cpart * P, nblk - 1) * 256 + 128 * h) / group, G - 1);
                    const int src = (c + 16 * (2 * u + h)) << 2;  // the lane that loaded group (u, h)
                    const uint32_t zw = FMT == 0 ? 0u : (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)zpr[t]);
                    const float zc = (float)(128 + F::zero_of(zw, gi));
                    const float sv = F::scale_of((uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)scr[t]));
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[t][e] += sv * (d[e] - zc * dx[h][e]);
                }
            }
        }
    }

    // wavefront w's tile t: D[i][c] at 4 (c + 16 (i / 4)) + i % 4 (lane c + 16 (i / 4), element i % 4)
    __shared__ __attribute__((aligned(16))) float red[NWK][NT][256];
#pragma unroll
    for (int t = 0; t < NT; ++t) *reinterpret_cast<v4f *>(&red[wave][t][4 * lane]) = acc[t];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < EL; ++i) {
        const Coord e = coord(i);
        const int n = nbase + TR * e.t + e.r;
        if (e.t >= RT || n >= N || e.b >= B) continue;
        float av = 0.f, uv = 0.f;  // summed over wavefronts, then parts, in that fixed order
#pragma unroll
        for (int w = 0; w < NWK; ++w)
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int ii = TR * s + e.b, cc = TR * s + e.r;
                const int at = 4 * (cc + 16 * (ii >> 2)) + (ii & 3);
                const float va = red[w][e.t][at], vu = EPI == EPI_SWIGLU ? red[w][NT - RT + e.t][at] : 0.f;
                av = (w == 0 && s == 0) ? va : av + va;
                uv = (w == 0 && s == 0) ? vu : uv + vu;
            }
        y[(size_t)e.b * N + n] = (uint16_t)f2bf(epi_value(EPI, av, uv, hr[i]));
    }
}

// ------------------------------------------------------------------------------------------------ dispatch
template <int FMT, int EPI>
void launch_w4_b1(const uint8_t *W, const void *S, const int32_t *Z, const uint16_t *x, uint16_t *y, int N, int K,
                  int group, hipStream_t st) {
    // wavefronts per CU: 4 up to 3072 rows (each wavefront amortizes its activation repack over more rows), 16 from
    // 32768 rows (more loads in flight on a long stream), else 8; the LFM2Q_W4_WPC knob overrides it
    const int wpc_env = knob_int(KNOB_W4_WPC, 0);
    const long wrows = (EPI == EPI_SWIGLU ? 2L : 1L) * N;
    const int wpc = wpc_env > 0 ? wpc_env : wrows <= 3072 ? 4 : wrows >= 32768 ? 16 : 8;
    const int C = K / 32;
    const int blocks = std::min((N + 3) / 4, std::max(1, device_cus() * wpc / 4));
    const dim3 grid(blocks);
    // one-shot (two rows per wavefront) below 32768 weight rows; the LFM2Q_W4_ONESHOT knob = 0 / 1 forces the
    // persistent / one-shot kernel
    bool oneshot = wrows < 32768;
    if (const KnobVal f = knob(KNOB_W4_ONESHOT); f.n) oneshot = f.v[0] != 0;
    if (oneshot && C <= 256) {
        const dim3 go((N + 7) / 8);
        // the activation repack shared by the workgroup for w1|w3 + SwiGLU and the residual GEMVs of K <= 2048
        // (LFM2Q_GEMV_XS = 0 / 1 forces it off / on). Measured on MI355X: each decode kind is faster with it in a
        // graph of that kind alone (w1|w3 5.41 -> 5.17 us, o/out_proj 3.83 -> 3.71, w2 4.62 -> 4.50, qkv 3.79 ->
        // 3.71), but in the 65-kernel decode step it on qkv / in_proj or on w2 lengthened the step by ~2.5 us while
        // shortening the kernels (a kernel trace shows the time moving into the gaps between kernels; not
        // understood), and on w1|w3 or o/out_proj alone it is neutral to -0.4 us
        const int xs_forced = knob_int(KNOB_GEMV_XS, -1);
        const bool xs = xs_forced >= 0 ? xs_forced == 1 : EPI == EPI_SWIGLU || (EPI == EPI_RESIDUAL && C <= 64);
#define LFM2Q_W4O(C_)                                                                                 \
    do {                                                                                              \
        if (xs)                                                                                       \
            gemv_w4_b1o_kernel<FMT, C_, EPI, 2, true><<<go, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N); \
        else                                                                                          \
            gemv_w4_b1o_kernel<FMT, C_, EPI, 2><<<go, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N);   \
    } while (0)
        if (C <= 64)
            LFM2Q_W4O(1);
        else if (C <= 128)
            LFM2Q_W4O(2);
        else
            LFM2Q_W4O(4);
#undef LFM2Q_W4O
        return;
    }
    if (C <= 64)
        gemv_w4_b1_kernel<FMT, 1, EPI><<<grid, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N);
    else if (C <= 128)
        gemv_w4_b1_kernel<FMT, 2, EPI><<<grid, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N);
    else
        gemv_w4_b1_kernel<FMT, 4, EPI><<<grid, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N);
}

// Launch shape from (weight rows, K, B) only -- a plain and a fused call over the same weights (w1|w3 as one
// [2 S, K/8] matrix) then split K alike, which keeps the fused epilogues bit-identical:
//   KS = 2 (8-row tiles) for batches up to 8 and at most 2048 weight rows; RT = 2 for 6144+ weight rows unless
//   KS = 2 or SwiGLU at batches up to 8, RT = 4 (at most 4 wavefronts) for 32768+ rows without SwiGLU (the lm_head,
//   batch 8: 27.9 -> 26.6 us);
//   NWK from the 256-k blocks per wavefront: 2 (4 when KS = 2, with at least 4 wavefronts past K = 2048), at most 8
//   wavefronts for two-tile workgroups and 16 otherwise. INT4 costs twice the VALU work per weight byte
//   of INT8, so its wavefronts take half the blocks (measured on MI355X at batches 2, 4 and 8). The
//   LFM2Q_W4_MFMA knob = "KS,RT,NWK" overrides the shape.
template <int FMT, int EPI, int KS, int RT>
void launch_w4_shape(const uint8_t *W, const void *S, const int32_t *Z, const uint16_t *x, uint16_t *y, int B, int N,
                     int K, int group, int nwk, hipStream_t st) {
    const dim3 grid((N + (16 / KS) * RT - 1) / ((16 / KS) * RT));
#define LFM2Q_W4M(NWK_) \
    gemv_w4_mfma_kernel<FMT, KS, RT, NWK_, EPI><<<grid, 64 * NWK_, 0, st>>>(W, S, Z, x, y, B, N, K, group, N)
    switch (nwk) {
        case 16: LFM2Q_W4M(16); break;
        case 8: LFM2Q_W4M(8); break;
        case 4: LFM2Q_W4M(4); break;
        case 2: LFM2Q_W4M(2); break;
        default: LFM2Q_W4M(1); break;
    }
#undef LFM2Q_W4M
}

template <int FMT, int EPI>
void launch_w4_mfma(const uint8_t *W, const void *S, const int32_t *Z, const uint16_t *x, uint16_t *y, int B, int N,
                    int K, int group, hipStream_t st) {
    const long wrows = EPI == EPI_SWIGLU ? 2L * N : N;
    const int nblk = (K + 255) / 256;
    int ks = (B <= 8 && wrows <= 2048) ? 2 : 1;
    // two row tiles per workgroup from 6144 weight rows, except w1|w3 + SwiGLU up to batch 8, where one tile per
    // workgroup (twice the workgroups) measured faster: 8.4-8.9 -> 7.6-8.3 us at batches 2-8 (even at 16)
    int rt = (ks == 1 && wrows >= 6144 && !(EPI == EPI_SWIGLU && B <= 8)) ? 2 : 1;
    if (EPI != EPI_SWIGLU && ks == 1 && wrows >= 32768) rt = 4;  // the lm_head: four tiles share each activation load
    const int bpw = ks == 2 ? 4 : 2;  // target blocks per wavefront
    int nwk = 1;
    // at most 8 wavefronts with two tiles pairs (16 would cap the registers at 128 and spill); 8-row tiles keep at
    // least 4 wavefronts past 2048 k (2 for K = 2048: the narrow o / out_proj kernels, measured at batch 8)
    while (nwk < (rt == 2 ? 8 : 16) && (nblk >= bpw * 2 * nwk || (ks == 2 && nblk > 8 && nwk < 4))) nwk *= 2;
    if (const KnobVal f = knob(KNOB_W4_MFMA); f.n == 3) {
        const int fk = f.v[0], fr = f.v[1], fn = f.v[2];
        if ((fk == 1 || (fk == 2 && B <= 8 && fr == 1)) &&
            (fr == 1 || fr == 2 || (fr == 4 && fk == 1 && EPI != EPI_SWIGLU)) &&
            (fn == 1 || fn == 2 || fn == 4 || fn == 8 || fn == 16)) {
            ks = fk;
            rt = fr;
            nwk = fn;
        }
    }
    if constexpr (EPI != EPI_SWIGLU) {
        if (rt == 4) {
            launch_w4_shape<FMT, EPI, 1, 4>(W, S, Z, x, y, B, N, K, group, std::min(nwk, 4), st);
            return;
        }
    }
    if (ks == 2)
        launch_w4_shape<FMT, EPI, 2, 1>(W, S, Z, x, y, B, N, K, group, nwk, st);
    else if (rt == 2)
        launch_w4_shape<FMT, EPI, 1, 2>(W, S, Z, x, y, B, N, K, group, nwk, st);
    else
        launch_w4_shape<FMT, EPI, 1, 1>(W, S, Z, x, y, B, N, K, group, nwk, st);
}

template <int FMT, int EPI>
void w4_run(const uint8_t *W, const void *S, const int32_t *Z, const uint16_t *x, uint16_t *y, int B, int N, int K,
            int group, hipStream_t st) {
    for (int b0 = 0; b0 < B; b0 += 16) {
        const int bs = std::min(16, B - b0);
        const uint16_t *xb = x + (size_t)b0 * K;
        uint16_t *yb = y + (size_t)b0 * N;
        const bool b1_mfma = knob_int(KNOB_W4_B1_MFMA, 0) != 0;
        if ((bs > 1 || b1_mfma) && group % 128 == 0) {
            launch_w4_mfma<FMT, EPI>(W, S, Z, xb, yb, bs, N, K, group, st);
        } else {
            for (int b = 0; b < bs; ++b)
                launch_w4_b1<FMT, EPI>(W, S, Z, xb + (size_t)b * K, yb + (size_t)b * N, N, K, group, st);
        }
    }
}

}  // namespace
}  // namespace lfm2q

using namespace lfm2q;

extern "C" int lfm2q_gemv_w4(int fmt, const void *Wq, const void *S, const int32_t *Z, const lfm2q_bf16 *x,
                             lfm2q_bf16 *y, int B, int N, int K, int group, int epi, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(fmt == 0 || fmt == 1, LFM2Q_ERR_ARG, "gemv_w4: fmt must be 0 (uint8 + fp32 scales) or 1 (int32 + "
                  "fp16 scales + zero points), got %d", fmt);
    LFM2Q_REQUIRE(epi >= 0 && epi <= 2, LFM2Q_ERR_ARG, "gemv_w4: epi must be 0 (none), 1 (SwiGLU) or 2 (residual)");
    LFM2Q_REQUIRE(Wq && S && x && y, LFM2Q_ERR_ARG, "gemv_w4: null pointer");
    LFM2Q_REQUIRE(fmt == 0 || Z, LFM2Q_ERR_ARG, "gemv_w4: fmt 1 needs zero points");
    LFM2Q_REQUIRE(B >= 1 && N >= 1 && K >= 32, LFM2Q_ERR_SHAPE, "gemv_w4: x [B, K], y [B, N] (B=%d N=%d K=%d)", B, N,
                  K);
    LFM2Q_REQUIRE(group >= 32 && group % 32 == 0 && K % group == 0, LFM2Q_ERR_SHAPE,
                  "gemv_w4: group size must be a multiple of 32 dividing K (group=%d K=%d)", group, K);
    LFM2Q_REQUIRE(K <= 8192, LFM2Q_ERR_SHAPE, "gemv_w4: K <= 8192 (K=%d)", K);
    LFM2Q_REQUIRE(aligned16(Wq) && aligned16(x), LFM2Q_ERR_ALIGN, "gemv_w4: Wq and x must be 16-byte aligned");
    const uint8_t *W = reinterpret_cast<const uint8_t *>(Wq);
    const hipStream_t st = (hipStream_t)stream;
#define LFM2Q_W4RUN(F_, E_) w4_run<F_, E_>(W, S, Z, x, y, B, N, K, group, st)
    if (fmt == 0) {
        if (epi == 0) LFM2Q_W4RUN(0, EPI_NONE);
        else if (epi == 1) LFM2Q_W4RUN(0, EPI_SWIGLU);
        else LFM2Q_W4RUN(0, EPI_RESIDUAL);
    } else {
        if (epi == 0) LFM2Q_W4RUN(1, EPI_NONE);
        else if (epi == 1) LFM2Q_W4RUN(1, EPI_SWIGLU);
        else LFM2Q_W4RUN(1, EPI_RESIDUAL);
    }
#undef LFM2Q_W4RUN
    return launch_status("gemv_w4");
}
