// W8A8 GEMM for gfx950: Y[M, N] = epilogue( Xq[M, K] . Wq[N, K]^T ), int8 x int8 -> exact int32 on the matrix
// cores (v_mfma_i32_32x32x32_i8), then either the int32 accumulators themselves or the per-token / per-channel
// dequant epilogue y = bf16( gelu?( ((float)acc * sx[m]) * sw[n] + b[n] ) ) with three separately rounded fp32 ops.
//
// Tiling: a 256-thread workgroup (4 wavefronts as 2 x 2) owns a BM x BN output tile; each wavefront a
// (BM/2) x (BN/2) block of 32 x 32 MFMA tiles. K advances in 64-byte stages through two LDS buffers: the global
// loads of stage s + 1 are in flight (in registers) while the MFMAs of stage s run, then land in the other buffer.
// LDS rows are 64 bytes (4 chunks of 16); chunk c of row r is stored at slot c ^ ((r >> 1) & 3), so the 8 rows a
// ds_read_b128 phase reads at one logical chunk, and the 8 chunks a ds_write_b128 phase writes, fall in 8 distinct
// 16-byte bank groups. M, N and K tails are zero-filled at load time (K % 16 == 0); stores are predicated.
//
// Activation quantization is its own memory-bound kernel (quant_rows_kernel): quantizing inside the GEMM's main
// loop would redo the per-element VALU work once per N tile, about twice the MFMA time of the tile.
//
// Reference: kernels/int8_gemm.cu:125-297 (gemm_i8_kernel, per-token path), :93-115 (store_tile epilogue),
// :391-432 (quant_rows_kernel), :690-702 (pick_bm); bound as gemm_i8 / quant_rows in kernels/int8_gemm.cpp.
#include "common.hpp"
#include "status.hpp"

#include <algorithm>

namespace lfm2q {
namespace {

constexpr int GT = 256;  // threads per GEMM workgroup
constexpr int BK = 64;   // bytes of K per stage

__device__ __forceinline__ int swz(int r, int c) { return (r * 4 + (c ^ ((r >> 1) & 3))) * 16; }

enum GemmOut { OUT_BF16 = 0, OUT_BF16_GELU = 1, OUT_I32 = 2 };

// ((float)acc * sx) * sw + b, each op rounded separately (no FMA contraction), then optional GELU
__device__ __forceinline__ float dequant(int acc, float sx, float sw, float b) {
#pragma clang fp contract(off)
    float v = (float)acc * sx;
    v = v * sw;
    return v + b;
}

template <int BM, int BN, int OUT>
__global__ __launch_bounds__(GT) void gemm_i8_kernel(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                     const float *__restrict__ sx, const float *__restrict__ sw,
                                                     const uint16_t *__restrict__ bias, void *__restrict__ Y, int M,
                                                     int N, int K) {
    constexpr int WM = BM / 2, WN = BN / 2;     // wavefront block
    constexpr int TM = WM / 32, TN = WN / 32;   // 32 x 32 MFMA tiles per wavefront
    constexpr int LA = BM * 4 / GT, LB = BN * 4 / GT;  // 16-byte global loads per thread per stage
    static_assert(LA >= 1 && LB >= 1 && TM >= 1 && TN >= 1, "tile too small");
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * BK];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * BK];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int KT = (K + BK - 1) / BK;

    // global -> register staging: thread t moves chunk (row = t / 4 + 64 j, c = t % 4) of each operand tile
    v4i ra[LA], rb[LB];
    auto gload = [&](int kt) {
        const int k = kt * BK + (tid & 3) * 16;
#pragma unroll
        for (int j = 0; j < LA; ++j) {
            const int r = (tid >> 2) + 64 * j, gm = m0 + r;
            ra[j] = (gm < M && k < K) ? ld16(A + (size_t)gm * K + k) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < LB; ++j) {
            const int r = (tid >> 2) + 64 * j, gn = n0 + r;
            rb[j] = (gn < N && k < K) ? ld16(B + (size_t)gn * K + k) : v4i{0, 0, 0, 0};
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int j = 0; j < LA; ++j)
            *reinterpret_cast<v4i *>(sA[buf] + swz((tid >> 2) + 64 * j, tid & 3)) = ra[j];
#pragma unroll
        for (int j = 0; j < LB; ++j)
            *reinterpret_cast<v4i *>(sB[buf] + swz((tid >> 2) + 64 * j, tid & 3)) = rb[j];
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    gload(0);
    swrite(0);
    __syncthreads();
    const int lr = lane & 31, lh = lane >> 5;  // MFMA operand row / k-half of this lane
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        const bool next = kt + 1 < KT;
        if (next) gload(kt + 1);
        const uint8_t *a_s = sA[buf], *b_s = sB[buf];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {  // two 32-byte k steps per stage
            const int c = 2 * kk + lh;
            v4i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const v4i *>(a_s + swz(wm * WM + 32 * i + lr, c));
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const v4i *>(b_s + swz(wn * WN + 32 * j + lr, c));
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (next) swrite(buf ^ 1);
        __syncthreads();
    }

    // epilogue. 32x32 MFMA output: lane l, element e -> row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * WN + 32 * j + lr;
        if (n >= N) continue;
        float w = 0.f, b = 0.f;
        if (OUT != OUT_I32) {
            w = sw[n];
            b = bias ? bf2f(bias[n]) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * WM + 32 * i + 8 * (e >> 2) + 4 * lh + (e & 3);
                if (m >= M) continue;
                if (OUT == OUT_I32) {
                    reinterpret_cast<int32_t *>(Y)[(size_t)m * N + n] = acc[i][j][e];
                } else {
                    float v = dequant(acc[i][j][e], sx[m], w, b);
                    if (OUT == OUT_BF16_GELU) v = gelu_tanh_f32(v);
                    reinterpret_cast<uint16_t *>(Y)[(size_t)m * N + n] = (uint16_t)f2bf(v);
                }
            }
    }
}

// ------------------------------------------------------------------------------------------------ quant_rows
// One wavefront per row: s = max(amax, 1e-8) / 127 (IEEE division), q = clamp(rint(x / s), -127, 127) with
// round-half-even. x / s is evaluated as x * (1 / s) unless that product lies within 2^-12 of a half-integer,
// where the correctly rounded quotient is computed instead: |x / s| <= 127 keeps the product within 2 ulp
// (< 2^-15) of the true quotient, so outside that band both round to the same integer and the result is the
// true-division one bit for bit.
__device__ __forceinline__ int quant1(float v, float s, float r) {
    float t = v * r;
    const float f = t - floorf(t);
    if (fabsf(f - 0.5f) < 0.000244140625f) t = v / s;
    return (int)fminf(fmaxf(rintf(t), -127.f), 127.f);
}

// 8 bf16 (one 16-byte vector) -> 8 int8 packed in two dwords
__device__ __forceinline__ void quant8(v4i xv, float s, float r, int &lo, int &hi) {
    int q[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        q[2 * j] = quant1(bf2f_lo((uint32_t)xv[j]), s, r);
        q[2 * j + 1] = quant1(bf2f_hi((uint32_t)xv[j]), s, r);
    }
    lo = (q[0] & 255) | ((q[1] & 255) << 8) | ((q[2] & 255) << 16) | ((q[3] & 255) << 24);
    hi = (q[4] & 255) | ((q[5] & 255) << 8) | ((q[6] & 255) << 16) | ((q[7] & 255) << 24);
}

__device__ __forceinline__ float absmax8(v4i xv, float m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf2f_lo((uint32_t)xv[j])), fabsf(bf2f_hi((uint32_t)xv[j]))));
    return m;
}

// rows of K bf16, K % 8 == 0. CH > 0: K = 512 CH exactly, the row stays in registers (CH 16-byte vectors per lane);
// CH == 0: any K, two passes over the row (the second one hits the cache).
template <int CH>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t *__restrict__ x, int8_t *__restrict__ q,
                                                         float *__restrict__ s, int rows, int K) {
    const int lane = threadIdx.x & 63;
    const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (row >= rows) return;
    const uint16_t *xr = x + (size_t)row * K;
    int8_t *qr = q + (size_t)row * K;
    if constexpr (CH > 0) {
        v4i v[CH];
        float m = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = ld_nt16(xr + (size_t)(c * 64 + lane) * 8);
#pragma unroll
        for (int c = 0; c < CH; ++c) m = absmax8(v[c], m);
        const float sc = fmaxf(wave_max(m), 1e-8f) / 127.f, rc = 1.f / sc;
        if (lane == 0) s[row] = sc;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            int lo, hi;
            quant8(v[c], sc, rc, lo, hi);
            *reinterpret_cast<int2 *>(qr + (size_t)(c * 64 + lane) * 8) = make_int2(lo, hi);
        }
    } else {
        const int C = K / 8;
        float m = 0.f;
        for (int c = lane; c < C; c += 64) m = absmax8(ld16(xr + (size_t)c * 8), m);
        const float sc = fmaxf(wave_max(m), 1e-8f) / 127.f, rc = 1.f / sc;
        if (lane == 0) s[row] = sc;
        for (int c = lane; c < C; c += 64) {
            int lo, hi;
            quant8(ld16(xr + (size_t)c * 8), sc, rc, lo, hi);
            *reinterpret_cast<int2 *>(qr + (size_t)c * 8) = make_int2(lo, hi);
        }
    }
}

// ------------------------------------------------------------------------------------------------ dispatch
// Tile choice: the largest of 256x256, 256x128, 128x256, 128x128, 128x64, 64x64 (BM x BN) whose tile count fills the
// chip at least ~1.5 times over, else the one with the best balance of rounds x tile work.
struct TileCfg {
    int bm, bn;
};

inline TileCfg pick_tile(int M, int N, int K) {
    static const int force_bm = env_int("LFM2Q_GEMM_BM", 0), force_bn = env_int("LFM2Q_GEMM_BN", 0);
    const TileCfg opts[] = {{256, 256}, {256, 128}, {128, 256}, {128, 128}, {128, 64}, {64, 64}};
    if (force_bm && force_bn)
        for (const TileCfg &o : opts)
            if (o.bm == force_bm && o.bn == force_bn) return o;
    const int cus = device_cus();
    // estimated time ~ rounds * (tile MACs / per-CU rate + per-tile overhead), per-tile overhead ~ 4 stages of K
    double best = 1e30;
    TileCfg bestc = opts[0];
    for (const TileCfg &o : opts) {
        const long tiles = (long)((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn);
        const long rounds = (tiles + cus - 1) / cus;
        const double kst = (double)(K + BK - 1) / BK;
        // a 64x64 tile runs its MFMAs at about half the efficiency of 256x256 (LDS reads per MAC double as tiles
        // halve); model it as cost per stage ~ bm * bn * (1 + 64 / bm + 64 / bn) / 256^2
        const double stage = (double)o.bm * o.bn * (1.0 + 64.0 / o.bm + 64.0 / o.bn) / 65536.0;
        const double t = rounds * (kst + 4.0) * stage;
        if (t < best * 0.999) {
            best = t;
            bestc = o;
        }
    }
    return bestc;
}

template <int OUT>
void launch_gemm(const int8_t *A, const int8_t *B, const float *sx, const float *sw, const uint16_t *bias, void *Y,
                 int M, int N, int K, hipStream_t st) {
    const TileCfg t = pick_tile(M, N, K);
    const dim3 grid((N + t.bn - 1) / t.bn, (M + t.bm - 1) / t.bm);
#define LFM2Q_GEMM(BM_, BN_)                                                                                        \
    if (t.bm == BM_ && t.bn == BN_) {                                                                                \
        gemm_i8_kernel<BM_, BN_, OUT><<<grid, GT, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K);                         \
        return;                                                                                                      \
    }
    LFM2Q_GEMM(256, 256)
    LFM2Q_GEMM(256, 128)
    LFM2Q_GEMM(128, 256)
    LFM2Q_GEMM(128, 128)
    LFM2Q_GEMM(128, 64)
    LFM2Q_GEMM(64, 64)
#undef LFM2Q_GEMM
}

int check_gemm(const char *name, const int8_t *A, const int8_t *B, const void *Y, int M, int N, int K) {
    LFM2Q_REQUIRE(A && B && Y, LFM2Q_ERR_ARG, "%s: null pointer", name);
    LFM2Q_REQUIRE(M >= 1 && N >= 1 && K >= 16, LFM2Q_ERR_SHAPE, "%s: need M, N >= 1 and K >= 16 (M=%d N=%d K=%d)",
                  name, M, N, K);
    LFM2Q_REQUIRE(K % 16 == 0, LFM2Q_ERR_SHAPE, "%s: need K %% 16 == 0 (K=%d)", name, K);
    LFM2Q_REQUIRE(M <= 65535 * 64, LFM2Q_ERR_SHAPE, "%s: M too large (%d)", name, M);
    LFM2Q_REQUIRE(aligned16(A) && aligned16(B), LFM2Q_ERR_ALIGN, "%s: A and B must be 16-byte aligned", name);
    return LFM2Q_OK;
}

}  // namespace
}  // namespace lfm2q

using namespace lfm2q;

extern "C" int lfm2q_gemm_i8(const int8_t *A, const float *sa, const int8_t *B, const float *sb, const lfm2q_bf16 *bias,
                             lfm2q_bf16 *Y, int M, int N, int K, int gelu, lfm2q_stream_t stream) {
    if (int st = check_gemm("gemm_i8", A, B, Y, M, N, K)) return st;
    LFM2Q_REQUIRE(sa && sb, LFM2Q_ERR_ARG, "gemm_i8: sx and sw are required");
    if (gelu)
        launch_gemm<OUT_BF16_GELU>(A, B, sa, sb, bias, Y, M, N, K, (hipStream_t)stream);
    else
        launch_gemm<OUT_BF16>(A, B, sa, sb, bias, Y, M, N, K, (hipStream_t)stream);
    return launch_status("gemm_i8");
}

extern "C" int lfm2q_gemm_i8_i32(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K,
                                 lfm2q_stream_t stream) {
    if (int st = check_gemm("gemm_i8_i32", A, B, C, M, N, K)) return st;
    launch_gemm<OUT_I32>(A, B, nullptr, nullptr, nullptr, C, M, N, K, (hipStream_t)stream);
    return launch_status("gemm_i8_i32");
}

extern "C" int lfm2q_quant_rows(const lfm2q_bf16 *x, int8_t *q, float *s, int rows, int K, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(x && q && s, LFM2Q_ERR_ARG, "quant_rows: null pointer");
    LFM2Q_REQUIRE(rows >= 1 && K >= 8 && K % 8 == 0, LFM2Q_ERR_SHAPE,
                  "quant_rows: K must be a multiple of 8 (rows=%d K=%d)", rows, K);
    LFM2Q_REQUIRE(aligned16(x) && ((uintptr_t)q & 7) == 0, LFM2Q_ERR_ALIGN,
                  "quant_rows: x must be 16-byte and q 8-byte aligned");
    const dim3 grid((rows + 3) / 4);
    hipStream_t st = (hipStream_t)stream;
    switch (K % 512 == 0 ? K / 512 : 0) {
        case 1: quant_rows_kernel<1><<<grid, 256, 0, st>>>(x, q, s, rows, K); break;
        case 2: quant_rows_kernel<2><<<grid, 256, 0, st>>>(x, q, s, rows, K); break;
        case 4: quant_rows_kernel<4><<<grid, 256, 0, st>>>(x, q, s, rows, K); break;
        case 8: quant_rows_kernel<8><<<grid, 256, 0, st>>>(x, q, s, rows, K); break;
        case 16: quant_rows_kernel<16><<<grid, 256, 0, st>>>(x, q, s, rows, K); break;
        default: quant_rows_kernel<0><<<grid, 256, 0, st>>>(x, q, s, rows, K); break;
    }
    return launch_status("quant_rows");
}
