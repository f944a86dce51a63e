// INT4 weight-only decode GEMVs for gfx950: y[b, n] = sum_k s[n, g(k)] (q[n, k] - z[n, g(k)]) x[b, k], fp32
// accumulation, bf16 out, with the SwiGLU / residual epilogues of the INT8 GEMVs.
//
// Two weight formats, one nibble order (nibble i of 32-bit word w of a row holds weight k = 8 w + i):
//   fmt 0, the reference's: Wq uint8 [N, K/2] (weight 2j in the low nibble of byte j, stored as q + 8), scales
//          fp32 [N, K/group], zero point 8 for every group;
//   fmt 1, GPTQ-style:      Wq int32 [N, K/8], scales fp16 [N, K/group], zero points int32 [N, ceil(G/8)]
//          (nibble j of word w = zero point of group 8 w + j).
//
// Dequantization costs two bit operations per weight pair: ((word >> 4p) & 0x000F000F) | 0x43004300 is the bf16 pair
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

namespace lfm2q {
namespace {

enum Epi { EPI_NONE = 0, EPI_SWIGLU = 1, EPI_RESIDUAL = 2 };

// (128 + q[p], 128 + q[p + 4]) as a bf16 pair, p = 0..3, from one 8-weight word
__device__ __forceinline__ uint32_t w4pair(uint32_t w, int p) { return ((w >> (4 * p)) & 0x000F000Fu) | 0x43004300u; }

// (x[p], x[p + 4]) from 8 bf16 activations x0..x7 held as 4 dwords (x0 | x1 << 16, ...)
__device__ __forceinline__ uint32_t xpair(const v4i &d, int p) {
    const uint32_t lo = (uint32_t)d[p >> 1], hi = (uint32_t)d[2 + (p >> 1)];
    return __builtin_amdgcn_perm(hi, lo, (p & 1) ? 0x07060302u : 0x05040100u);
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2bf as_bf16x2(uint32_t v) { return __builtin_bit_cast(v2bf, v); }
__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// group scale and zero point of weight row `row`, group g
template <int FMT>
struct W4Fmt;
template <>
struct W4Fmt<0> {
    __device__ static float scale(const void *S, const int32_t *, int row, int g, int G) {
        return reinterpret_cast<const float *>(S)[(size_t)row * G + g];
    }
    __device__ static int zero(const int32_t *, int, int, int) { return 8; }
};
template <>
struct W4Fmt<1> {
    __device__ static float scale(const void *S, const int32_t *, int row, int g, int G) {
        return h2f(reinterpret_cast<const uint16_t *>(S)[(size_t)row * G + g]);
    }
    __device__ static int zero(const int32_t *Z, int row, int g, int G) {
        return ((uint32_t)Z[(size_t)row * ((G + 7) >> 3) + (g >> 3)] >> (4 * (g & 7))) & 15;
    }
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
    constexpr int NROW = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int NB = CPL * NROW <= 2 ? 4 : 2;
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * 4;
    const int G = K / group, C = K / 32;
    int n = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (n >= N) return;  // no block-level synchronization in this kernel

    int gl[CPL];  // group of the lane's chunk u (clamped for chunks past K)
#pragma unroll
    for (int u = 0; u < CPL; ++u) gl[u] = min(32 * (lane + 64 * u) / group, G - 1);
    const uint32_t rowb = (uint32_t)K / 2;
    struct Item {
        v4i w[CPL][NROW];
        float s[CPL][NROW];
        int z[CPL][NROW];
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
                it.s[u][i] = F::scale(S, Z, wc, gl[u], G);
                it.z[u][i] = F::zero(Z, wc, gl[u], G);
            }
        }
        if (EPI == EPI_RESIDUAL) it.h = y[rc];
    };
    // the first rows' weights are requested before the activations are repacked, so the two memory latencies
    // overlap instead of adding up
    Item buf[NB];
#pragma unroll
    for (int j = 0; j < NB - 1; ++j) load(buf[j], n + j * nw);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t xp[CPL][16];  // activation pairs, word-major: xp[u][4 j + p] = (x[8 j + p], x[8 j + p + 4])
    float xs[CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
        const int c = lane + 64 * u;
        xs[u] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const v4i d = c < C ? ld16(x + (size_t)c * 32 + 8 * j) : v4i{0, 0, 0, 0};
#pragma unroll
            for (int p = 0; p < 4; ++p) xp[u][4 * j + p] = xpair(d, p);
#pragma unroll
            for (int e = 0; e < 4; ++e) xs[u] += bf2f_lo((uint32_t)d[e]) + bf2f_hi((uint32_t)d[e]);
        }
    }
    auto finish = [&](const Item &it, int row) {
        float acc[NROW];
#pragma unroll
        for (int i = 0; i < NROW; ++i) {
            acc[i] = 0.f;
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                float d = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        d = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w4pair((uint32_t)it.w[u][i][j], p)),
                                                            as_bf16x2(xp[u][4 * j + p]), d, false);
                acc[i] += it.s[u][i] * (d - (float)(128 + it.z[u][i]) * xs[u]);
            }
            acc[i] = wave_sum(acc[i]);
        }
        const float v = epi_value(EPI, acc[0], acc[NROW - 1], EPI == EPI_RESIDUAL ? it.h : 0u);
        if (lane == 0) y[row] = (uint16_t)f2bf(v);
    };
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

// ------------------------------------------------------------------------------------------------ batch 2..16
// WG = NWK wavefronts and 16 RT output rows (EPI_SWIGLU: plus the 16 RT matching w3 rows, NT = 2 RT tiles). K goes
// in steps of 128 (one group when group = 128; group % 128 == 0 keeps every step inside one group); wavefront w
// takes steps [w SPW, (w + 1) SPW), SPW = K / 128 / NWK, in stages of up to 4 steps whose loads are all issued
// first. In a step, lane (col = l % 16, kq = l / 16) loads the 32 weights k0 + 32 kq .. + 31 of row col of every
// tile (16 bytes) and the activations of batch row col at the same k. MFMA j (j = 0..3) takes word j of both:
// k-slot s of lane group kq is k = k0 + 32 kq + 8 j + perm(s), the same map for both operands.
// Activations are the A operand (batch x k), weights B (k x rows): D[batch][row] sits in lane row + 16 (batch / 4),
// element batch % 4, so a lane's scale and zero point are those of its single row col. A fifth MFMA per j with B = 1
// gives the step's activation sums in the same layout.
template <int FMT, int RT, int NWK, int EPI>
__global__ __launch_bounds__(64 * NWK) void gemv_w4_mfma_kernel(const uint8_t *__restrict__ Wq,
                                                                const void *__restrict__ S,
                                                                const int32_t *__restrict__ Z,
                                                                const uint16_t *__restrict__ x,
                                                                uint16_t *__restrict__ y, int B, int N, int K,
                                                                int group, int Sr) {
    using F = W4Fmt<FMT>;
    constexpr int NT = (EPI == EPI_SWIGLU ? 2 : 1) * RT;
    constexpr int U = 4;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 15, kq = lane >> 4;
    const int nbase = blockIdx.x * 16 * RT;
    const int G = K / group, steps = K / 128, spw = steps / NWK;
    const uint32_t rowb = (uint32_t)K / 2;
    int wrow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
        wrow[t] = (EPI == EPI_SWIGLU && t >= RT ? Sr : 0) + min(nbase + 16 * (t % RT) + col, N - 1);
    const bool xm = col < B;
    const uint16_t *xrow = x + (size_t)(xm ? col : 0) * K;
    const v8bf ones = __builtin_bit_cast(v8bf, v4u{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

    v4f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int s0 = wave * spw; s0 < (wave + 1) * spw; s0 += U) {
        v4i wv[U][NT], xv[U][4];
        float sc[U][NT];
        int zp[U][NT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = s0 + u;
            const bool in = st < (wave + 1) * spw;
            const int k = 128 * st + 32 * kq;
            const int g = min(128 * st / group, G - 1);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                wv[u][t] = in ? ld_nt16(Wq + (size_t)wrow[t] * rowb + k / 2) : v4i{0, 0, 0, 0};
                sc[u][t] = F::scale(S, Z, wrow[t], g, G);
                zp[u][t] = F::zero(Z, wrow[t], g, G);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[u][j] = (in && xm) ? ld16(xrow + k + 8 * j) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + u < (wave + 1) * spw) {
                v4f d[NT], dx = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < NT; ++t) d[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v8bf a = __builtin_bit_cast(
                        v8bf, v4u{xpair(xv[u][j], 0), xpair(xv[u][j], 1), xpair(xv[u][j], 2), xpair(xv[u][j], 3)});
                    dx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, dx, 0, 0, 0);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const uint32_t w = (uint32_t)wv[u][t][j];
                        const v8bf b = __builtin_bit_cast(v8bf, v4u{w4pair(w, 0), w4pair(w, 1), w4pair(w, 2), w4pair(w, 3)});
                        d[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, d[t], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float zc = (float)(128 + zp[u][t]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[t][e] += sc[u][t] * (d[t][e] - zc * dx[e]);
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
            uint16_t *yo = y + (size_t)m * N + n;
            const float v = epi_value(EPI, acc[t][i], EPI == EPI_SWIGLU ? acc[RT + t][i] : 0.f,
                                      EPI == EPI_RESIDUAL ? *yo : 0u);
            *yo = (uint16_t)f2bf(v);
        }
    }
}

// ------------------------------------------------------------------------------------------------ dispatch
template <int FMT, int EPI>
void launch_w4_b1(const uint8_t *W, const void *S, const int32_t *Z, const uint16_t *x, uint16_t *y, int N, int K,
                  int group, hipStream_t st) {
    static const int wpc = env_int("LFM2Q_W4_WPC", 8);
    const int C = K / 32;
    const int blocks = std::min((N + 3) / 4, std::max(1, device_cus() * wpc / 4));
    const dim3 grid(blocks);
    if (C <= 64)
        gemv_w4_b1_kernel<FMT, 1, EPI><<<grid, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N);
    else if (C <= 128)
        gemv_w4_b1_kernel<FMT, 2, EPI><<<grid, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N);
    else
        gemv_w4_b1_kernel<FMT, 4, EPI><<<grid, 256, 0, st>>>(W, S, Z, x, y, N, K, group, N);
}

// NWK: the smallest of 1, 2, 4, 8 dividing the 128-k steps with (16-row weight tiles) x NWK >= 4096, else the largest
// that divides: 2048+ wavefronts even when a SwiGLU workgroup holds two tiles (8 per CU, the streaming optimum). RT: 16-row tiles per workgroup, 4 for outputs of 32768+ rows
// (not with SwiGLU, whose tile pairs double the registers), else 1.
template <int FMT, int EPI>
void launch_w4_mfma(const uint8_t *W, const void *S, const int32_t *Z, const uint16_t *x, uint16_t *y, int B, int N,
                    int K, int group, hipStream_t st) {
    const int steps = K / 128;
    const int rt = (N >= 32768 && EPI != EPI_SWIGLU) ? 4 : 1;
    const int wgs = (N + 16 * rt - 1) / (16 * rt);
    // the split is chosen from K and the weight-row count alone, so a fused SwiGLU call (N outputs over 2N rows)
    // splits K like the plain GEMV of the same 2N rows, and its results are bit-identical to that GEMV + silu_mul
    const long tiles16 = ((EPI == EPI_SWIGLU ? 2L : 1L) * N + 15) / 16;
    int nwk = 1;
    for (int c = 1; c <= 8; c <<= 1)
        if (steps % c == 0) {
            nwk = c;
            if (tiles16 * c >= 4096) break;
        }
    const dim3 grid(wgs);
#define LFM2Q_W4M(RT_, NWK_)                                                                                         \
    gemv_w4_mfma_kernel<FMT, RT_, NWK_, EPI><<<grid, 64 * NWK_, 0, st>>>(W, S, Z, x, y, B, N, K, group, N)
    if constexpr (EPI != EPI_SWIGLU) {
        if (rt == 4) {
            switch (nwk) {
                case 8: LFM2Q_W4M(4, 8); break;
                case 4: LFM2Q_W4M(4, 4); break;
                case 2: LFM2Q_W4M(4, 2); break;
                default: LFM2Q_W4M(4, 1); break;
            }
            return;
        }
    }
    {
        switch (nwk) {
            case 8: LFM2Q_W4M(1, 8); break;
            case 4: LFM2Q_W4M(1, 4); break;
            case 2: LFM2Q_W4M(1, 2); break;
            default: LFM2Q_W4M(1, 1); break;
        }
    }
#undef LFM2Q_W4M
}

template <int FMT, int EPI>
void w4_run(const uint8_t *W, const void *S, const int32_t *Z, const uint16_t *x, uint16_t *y, int B, int N, int K,
            int group, hipStream_t st) {
    for (int b0 = 0; b0 < B; b0 += 16) {
        const int bs = std::min(16, B - b0);
        const uint16_t *xb = x + (size_t)b0 * K;
        uint16_t *yb = y + (size_t)b0 * N;
        if (bs > 1 && group % 128 == 0) {
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
