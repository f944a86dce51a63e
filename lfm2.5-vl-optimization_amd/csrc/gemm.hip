// W8A8 GEMM for gfx950 and its W8A16 sibling: Y[M, N] = epilogue( Xq[M, K] . Wq[N, K]^T ), int8 x int8 -> exact
// int32 on the matrix cores (v_mfma_i32_32x32x32_i8), then either the int32 accumulators themselves or the
// per-token / per-channel dequant epilogue y = bf16( gelu?( ((float)acc * sx[m]) * sw[n] + b[n] ) ) with three
// separately rounded fp32 ops (grouped-64 activation scales: the per-group fold of gemm_i8_kernel's GRP form; INT8
// output: requantized per 64 columns for the next GEMM).
//
// Kernels:
// - gemm_i8_kernel: one BM x BN tile per 256-thread workgroup (4 wavefronts as 2 x 2); operands go global -> LDS
//   directly (buffer_load ... lds) through an NSTG-deep ring of 64-byte stages; optionally K split over KSP
//   wavefront groups (exact int32 partials summed in LDS), the grouped fold (GRP), INT8 output, or bf16 activations
//   quantized on their way into LDS (XBF).
// - gemm_i8_big_kernel: 256 x 256 tiles on 8 wavefronts with BKT-byte stages.
// - gemm_i8_bigp_kernel: the persistent form (one workgroup per CU walks its tiles; the next tile's first stage and
//   epilogue operands load during the current tile's epilogue) in 256 x 256, 256 x 128, 128 x 128 and 128 x 64
//   tiles with 2-6 ring slots of 128-byte stages, optionally with K cut across workgroups through a workspace.
// - gemm_w8_kernel: W8A16, bf16 activations x int8 weights on the bf16 matrix cores.
// Which kernel and tile run is decided by the cost models of the dispatch section at the end of the file.
//
// M, N and K tails are zero-filled at load time by the buffer range check (K % 16 == 0); stores are predicated.
// Activation quantization is normally its own memory-bound kernel (quant.hip): the XBF form, which quantizes inside
// the main loop, redoes that per-element work once per N tile and measured 3-6x slower on the LFM2 / SigLIP2 shapes.
//
// Reference: kernels/int8_gemm.cu:125-297 (gemm_i8_kernel, per-token path), :93-115 (store_tile epilogue),
// :690-702 (pick_bm); bound as gemm_i8 in kernels/int8_gemm.cpp.
#include "common.hpp"
#include "quantize.hpp"
#include "status.hpp"

#include <algorithm>
#include <type_traits>

namespace lfm2q {
namespace {

constexpr int GT = 256;  // threads per GEMM workgroup
constexpr int BK = 64;   // bytes of K per stage

// LDS byte offset of 16-byte chunk c of 64-byte row r: chunk c is stored at slot c ^ ((r >> sh) & 3)
__device__ __forceinline__ int swz(int r, int c, int sh) { return (r * 4 + (c ^ ((r >> sh) & 3))) * 16; }

// bf16 out, bf16 out after GELU, the int32 accumulators, or INT8 + per-64-column scales (after GELU) for the next GEMM
enum GemmOut { OUT_BF16 = 0, OUT_BF16_GELU = 1, OUT_I32 = 2, OUT_Q8 = 3, OUT_Q8_GELU = 4 };
constexpr bool out_gelu(int o) { return o == OUT_BF16_GELU || o == OUT_Q8_GELU; }
constexpr bool out_q8(int o) { return o == OUT_Q8 || o == OUT_Q8_GELU; }

typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// per-token: ((float)acc * sx) * sw + b, each op rounded separately (no FMA contraction)
__device__ __forceinline__ float dequant(int acc, float sx, float sw, float b) {
#pragma clang fp contract(off)
    float v = (float)acc * sx;
    v = v * sw;
    return v + b;
}
// grouped: the fp32 accumulator already carries the activation scales; facc * sw + b
__device__ __forceinline__ float dequant(float facc, float, float sw, float b) {
#pragma clang fp contract(off)
    const float v = facc * sw;
    return v + b;
}


// Workgroup -> output tile. Workgroups are dealt to the 8 XCDs round-robin (workgroup w runs on XCD w % 8), so the
// tile sequence is split into 8 contiguous bands and band x is given to the workgroups of XCD x; inside the band
// tiles go in groups of 8 M-tiles that sweep N, so concurrently resident workgroups of one XCD share operand panels
// in that XCD's L2.
__device__ __forceinline__ void group_of(int t, int tm_n, int tn_n, int &tm, int &tn) {
    constexpr int GM = 8;
    const int per_group = GM * tn_n;
    const int g = t / per_group, r = t % per_group;
    const int gm = min(GM, tm_n - g * GM);
    tm = g * GM + r % gm;
    tn = r / gm;
}
__device__ __forceinline__ void tile_of(int w, int tm_n, int tn_n, int &tm, int &tn) {
    const int T = tm_n * tn_n;
    group_of(T % 8 == 0 ? (w % 8) * (T / 8) + w / 8 : w, tm_n, tn_n, tm, tn);
}

constexpr int STAGES = 3;  // LDS ring depth: stage s computes while s + 1 and s + 2 are loading
// The GEMM workspace: for the K split across workgroups (lfm2q_gemm_i8_ex / lfm2q_gemm_w8_ex) one arrival counter
// per output tile, then the partial accumulator tiles; after them the control block of the quantizing prologue
// (lfm2q_gemm_i8_fq), which the split never touches.
constexpr uint32_t SPLIT_CNT_WORDS = 16384;
constexpr size_t GEMM_SPLIT_BYTES = 4 * SPLIT_CNT_WORDS + (64u << 20);
constexpr size_t GEMM_CTL_BYTES = 65536 * 4;
constexpr size_t GEMM_WS_BYTES = GEMM_SPLIT_BYTES + GEMM_CTL_BYTES;

// s_waitcnt immediate for vmcnt(n) with the other counters at their maximum (gfx9: vmcnt bits 3:0 and 15:14)
constexpr int vmcnt_imm(int n) { return 0x3f70 | (n & 15) | ((n >> 4) << 14); }
// wait until at most `ahead` stages of PER loads each are outstanding (ahead <= 6)
template <int PER>
__device__ __forceinline__ void wait_stages(int ahead) {
    switch (ahead) {
        case 6: __builtin_amdgcn_s_waitcnt(vmcnt_imm(6 * PER)); break;
        case 5: __builtin_amdgcn_s_waitcnt(vmcnt_imm(5 * PER)); break;
        case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * PER)); break;
        case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * PER)); break;
        case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER)); break;
        case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER)); break;
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
    }
}

// f(kt + S, integral_constant<S>) for S = S0 .. N - 1: a loop body copied once per ring slot, so that each copy's
// slot is a compile-time constant
template <int S, int N, class F>
__device__ __forceinline__ void slot_steps(int kt, F &f) {
    if constexpr (S < N) {
        f(kt + S, std::integral_constant<int, S>{});
        slot_steps<S + 1, N>(kt, f);
    }
}
// the same for the stages below KT only (a ring's last, partial round)
template <int S, int N, class F>
__device__ __forceinline__ void slot_steps_below(int kt, int KT, F &f) {
    if constexpr (S < N) {
        if (kt + S < KT) f(kt + S, std::integral_constant<int, S>{});
        slot_steps_below<S + 1, N>(kt, KT, f);
    }
}

// Epilogue of one wavefront block: tokens mb .. mb + 32 TM - 1 x weight rows nb .. nb + 32 TN - 1. Per tile (i, j)
// and run q the lane holds 4 consecutive output columns n .. n + 3 of token row m.
template <int TM, int TN, int OUT, typename ACC>
__device__ __forceinline__ void store_tile(const ACC (&acc)[TN][TM], const float *__restrict__ sx,
                                           const float *__restrict__ sw, const uint16_t *__restrict__ bias,
                                           void *__restrict__ Y, int M, int N, int mb, int nb, int lr, int lh) {
    // 4-wide vector path: rows of 4k elements and aligned Y (16 B), sw (16 B) and bias (8 B)
    const bool vec = (N & 3) == 0 && (((uintptr_t)Y | (uintptr_t)sw) & 15) == 0 && ((uintptr_t)bias & 7) == 0;
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int m = mb + 32 * j + lr;
        if (m >= M) continue;
        const float s_m = (OUT == OUT_I32 || !sx) ? 0.f : sx[m];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = nb + 32 * i + 8 * q + 4 * lh;
                if (n >= N) continue;
                const size_t o = (size_t)m * N + n;
                if constexpr (OUT == OUT_I32) {
                    if (vec) {
                        *reinterpret_cast<v4i *>(reinterpret_cast<int32_t *>(Y) + o) =
                            v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < N) reinterpret_cast<int32_t *>(Y)[o + e] = acc[i][j][4 * q + e];
                    }
                } else {
                    float v[4];
                    if (vec) {
                        const v4f w4 = *reinterpret_cast<const v4f *>(sw + n);
                        uint32_t b01 = 0, b23 = 0;
                        if (bias) {
                            const uint2 bb = *reinterpret_cast<const uint2 *>(bias + n);
                            b01 = bb.x;
                            b23 = bb.y;
                        }
                        v[0] = dequant(acc[i][j][4 * q], s_m, w4[0], bf2f_lo(b01));
                        v[1] = dequant(acc[i][j][4 * q + 1], s_m, w4[1], bf2f_hi(b01));
                        v[2] = dequant(acc[i][j][4 * q + 2], s_m, w4[2], bf2f_lo(b23));
                        v[3] = dequant(acc[i][j][4 * q + 3], s_m, w4[3], bf2f_hi(b23));
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int ne = min(n + e, N - 1);
                            v[e] = dequant(acc[i][j][4 * q + e], s_m, sw[ne], bias ? bf2f(bias[ne]) : 0.f);
                        }
                    }
                    if (out_gelu(OUT))
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = gelu_tanh_f32(v[e]);
                    uint16_t *yo = reinterpret_cast<uint16_t *>(Y) + o;
                    if (vec) {
                        *reinterpret_cast<uint2 *>(yo) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < N) yo[e] = (uint16_t)f2bf(v[e]);
                    }
                }
            }
    }
}

// Staged epilogue for bf16 output, used when N % 8 == 0 and Y / sw are 16-byte (bias 8-byte) aligned. The MFMA
// layout leaves each lane with 16-byte pieces of 32 different token rows, which as direct stores become partial-line
// writes spread over rows N * 2 bytes apart. Instead each wavefront dequantizes one 32-token slice of its block at a
// time into its own LDS region (row pitch 2 WN + 8 bytes: conflict-free 8-byte writes of 32 rows), then reads it
// back row-major (two 8-byte reads per lane and row) and writes whole contiguous row runs, 16 bytes per lane. LDS ops of one wavefront execute in order,
// so the slice needs no barrier between its writes and the reads of other lanes, nor before the next slice.
template <int TN>
constexpr int stage_bytes() { return 32 * (64 * TN + 8); }

template <int TM, int TN, int OUT, typename ACC>
__device__ __forceinline__ void store_tile_staged(const ACC (&acc)[TN][TM], const float *__restrict__ sx,
                                                  const float *__restrict__ sw, const uint16_t *__restrict__ bias,
                                                  void *__restrict__ Y, float *__restrict__ YsT, int M, int N, int mb,
                                                  int nb, int lane, uint8_t *stage) {
    constexpr int WN = 32 * TN;      // output columns of the block
    constexpr int P = 2 * WN + 8;    // LDS row pitch (bytes)
    constexpr int CPRo = WN / 8;     // 16-byte chunks per output row
    constexpr int RPI = 64 / CPRo;   // rows per store instruction
    const int lr = lane & 31, lh = lane >> 5;
    const int c = lane % CPRo, r0 = lane / CPRo;
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int m = mb + 32 * j + lr;
        const float s_m = sx ? sx[min(m, M - 1)] : 0.f;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = min(nb + 32 * i + 8 * q + 4 * lh, N - 4);  // N % 8 == 0: clamped runs are whole
                const v4f w4 = *reinterpret_cast<const v4f *>(sw + n);
                uint32_t b01 = 0, b23 = 0;
                if (bias) {
                    const uint2 bb = *reinterpret_cast<const uint2 *>(bias + n);
                    b01 = bb.x;
                    b23 = bb.y;
                }
                float v[4];
                v[0] = dequant(acc[i][j][4 * q], s_m, w4[0], bf2f_lo(b01));
                v[1] = dequant(acc[i][j][4 * q + 1], s_m, w4[1], bf2f_hi(b01));
                v[2] = dequant(acc[i][j][4 * q + 2], s_m, w4[2], bf2f_lo(b23));
                v[3] = dequant(acc[i][j][4 * q + 3], s_m, w4[3], bf2f_hi(b23));
                if (out_gelu(OUT))
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = gelu_tanh_f32(v[e]);
                *reinterpret_cast<uint2 *>(stage + lr * P + 2 * (32 * i + 8 * q + 4 * lh)) =
                    make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int rr = 0; rr < 32; rr += RPI) {
            const int r = rr + r0;
            // two 8-byte reads: odd rows are only 8-byte aligned at this pitch
            const uint2 v0 = *reinterpret_cast<const uint2 *>(stage + r * P + 16 * c);
            const uint2 v1 = *reinterpret_cast<const uint2 *>(stage + r * P + 16 * c + 8);
            const int mo = mb + 32 * j + r, no = nb + 8 * c;
            if constexpr (out_q8(OUT)) {
                // the 8 lanes c0 .. c0 + 7 (c0 % 8 == 0) of this row hold one 64-column group of bf16 outputs:
                // quantize it exactly as quant_groups does
                const v4i xv = v4i{(int)v0.x, (int)v0.y, (int)v1.x, (int)v1.y};
                float am = absmax8(xv, 0.f);
                am = fmaxf(am, __shfl_xor(am, 1));
                am = fmaxf(am, __shfl_xor(am, 2));
                am = fmaxf(am, __shfl_xor(am, 4));
                const float sc = scale_of(am);
                if (mo < M && no < N) {
                    int lo, hi;
                    quant8(xv, sc, 1.f / sc, lo, hi);
                    *reinterpret_cast<int2 *>(reinterpret_cast<int8_t *>(Y) + (size_t)mo * N + no) = make_int2(lo, hi);
                    if ((c & 7) == 0) YsT[(size_t)(no >> 6) * M + mo] = sc;
                }
            } else if (mo < M && no < N) {
                *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(Y) + (size_t)mo * N + no) =
                    make_uint4(v0.x, v0.y, v1.x, v1.y);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// INT8 output always takes the staged path (its callers guarantee N % 64 == 0 and the alignments)
template <int TM, int TN, int OUT, typename ACC>
__device__ __forceinline__ void epilogue(const ACC (&acc)[TN][TM], const float *__restrict__ sx,
                                         const float *__restrict__ sw, const uint16_t *__restrict__ bias,
                                         void *__restrict__ Y, float *__restrict__ YsT, int M, int N, int mb, int nb,
                                         int lane, uint8_t *stage) {
    const int lr = lane & 31, lh = lane >> 5;
    if constexpr (out_q8(OUT)) {
        store_tile_staged<TM, TN, OUT>(acc, sx, sw, bias, Y, YsT, M, N, mb, nb, lane, stage);
    } else {
        if (OUT != OUT_I32 && (N & 7) == 0 && (((uintptr_t)Y | (uintptr_t)sw) & 15) == 0 &&
            ((uintptr_t)bias & 7) == 0)
            store_tile_staged<TM, TN, OUT>(acc, sx, sw, bias, Y, YsT, M, N, mb, nb, lane, stage);
        else
            store_tile<TM, TN, OUT>(acc, sx, sw, bias, Y, M, N, mb, nb, lr, lh);
    }
}

// BM: token rows (M) per workgroup, BN: weight rows (N). Wavefront (wm, wn) of the 2 x 2 grid owns BM/2 tokens x
// BN/2 weight rows as TN x TM tiles of 32 x 32, with the weights as the MFMA A operand and the tokens as B, so a
// lane's accumulator holds, per tile, 4 runs of 4 consecutive output columns of one token row: D[n][m], lane l ->
// m = l % 32, element e -> n = 8 (e / 4) + 4 (l / 32) + e % 4.
//
// Operand tiles go global -> LDS directly (buffer_load_dwordx4 ... lds): one wavefront instruction fills 1 KiB of
// LDS in lane order, i.e. 16 rows of 64 bytes, so lane i fetches the logical chunk c = (i % 4) ^ key(row) that the
// swizzled layout keeps in that slot. Rows past M and chunks past K read zeros (buffer range check). The loads of
// stage s + 2 are issued before the MFMAs of stage s; one s_waitcnt + barrier per stage makes stage s visible.
// GRP (grouped-64 activation scales, sx = sxT [K/64, M]): a 64-byte stage is one scale group. The stage's int32
// sums (the first k step starts from zero) are folded into fp32 accumulators after its MFMAs,
// facc = fma((float)acc, sxT[kt, m], facc), in stage order -- the reference's fold, exact per group since |acc| <=
// 64 * 127^2 < 2^24. The group's scales for the tile's rows travel with the operands (one 4-byte direct load per
// wavefront per stage into a 1 KiB LDS slot) and are read after the stage's barrier. YsT: OUT_Q8 scales.
// Occupancy hint: two wavefronts per SIMD, except where the 6-stage ring of a large tile (or the bf16 staging ring of
// a 128-row tile) leaves room for one workgroup, and three for the grouped kernel's tile-sequential fold (SEQ)
template <int BM, int BN, int NSTG, bool XBF = false, bool SEQ = false>
constexpr int gemm_waves_per_eu() {
    return SEQ ? 3 : (NSTG == 6 && BM + BN > 192) || (XBF && BM == 128) ? 1 : 2;
}

template <int BM, int BN, int OUT, bool GRP = false, int NSTG = STAGES, int KSP = 1, bool XBF = false, bool SEQ = false>
__global__ __launch_bounds__(GT * KSP) __attribute__((amdgpu_waves_per_eu(gemm_waves_per_eu<BM, BN, NSTG, XBF, SEQ>()))) void gemm_i8_kernel(
    const int8_t *__restrict__ X, const int8_t *__restrict__ W, const float *__restrict__ sx,
    const float *__restrict__ sw, const uint16_t *__restrict__ bias, void *__restrict__ Y, int M, int N, int K,
    int sh, float *__restrict__ YsT = nullptr) {
    constexpr int WMt = BM / 2, WNt = BN / 2;   // wavefront block: tokens x weight rows
    constexpr int TM = WMt / 32, TN = WNt / 32;  // 32 x 32 MFMA tiles per wavefront
    constexpr int IX = BM / 64, IW = BN / 64;    // direct-load instructions per wavefront per stage (16 rows each)
    constexpr int IS = GRP ? 1 : 0;               // scale loads per wavefront per stage
    static_assert(IX >= 1 && IW >= 1 && TM >= 1 && TN >= 1, "tile too small");
    static_assert(4 * stage_bytes<TN>() <= NSTG * (BM + BN) * BK, "epilogue staging exceeds the LDS ring");
    static_assert(!out_q8(OUT) || (GRP && WNt % 64 == 0), "INT8 output needs grouped input and 64-column blocks");
    // KSP > 1: KSP groups of 4 wavefronts split the K stages of one tile, each with its own operand ring; their
    // int32 accumulators meet in LDS at the end (exact, so the result does not depend on KSP). Per-token only: the
    // grouped path folds fp32 scales stage by stage, in order.
    static_assert(KSP == 1 || (!GRP && !out_q8(OUT)), "split K needs the int32 accumulators of the per-token path");
    static_assert(KSP == 1 || (KSP - 1) * BM * BN * 4 <= KSP * NSTG * (BM + BN) * BK, "partials exceed the rings");
    // XBF: X is bf16 [M, K] and sx its rows' quant_rows scales. Each stage's activations come global -> LDS by direct
    // loads (bf16, 128-byte rows) beside the weights, and each wavefront quantizes the rows it loaded itself
    // (quant8, the quantizers' own code) into the int8 slot the direct int8 loads would have filled.
    static_assert(!XBF || (!GRP && KSP == 1 && NSTG == 3 && BM <= 128), "bf16 activations: per-token, 3-stage ring");
    // SEQ: the grouped fold tile by tile through two int32 accumulator buffers (instead of every tile's), so that the
    // 128 x 128 kernel fits three wavefronts per SIMD; with a 3-stage ring three workgroups share a CU's LDS
    static_assert(!SEQ || (GRP && KSP == 1 && (TN * TM) % 2 == 0), "tile-sequential fold: grouped, even tile count");
    constexpr int IXB = XBF ? BM / 32 : 1;  // bf16 activation loads per wavefront per stage (8 rows x 128 bytes)
    constexpr int XBS = XBF ? NSTG * BM * 2 * BK : 0;  // bf16 staging ring
    constexpr int RING = NSTG * (BM + BN) * BK;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[KSP * RING + (GRP ? NSTG * 1024 : 0) + XBS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int grp = KSP == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid >> 8);  // K group of this wavefront
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);         // wavefront within its group
    const int wm = wave >> 1, wn = wave & 1;
    uint8_t(*sX)[BM * BK] = reinterpret_cast<uint8_t(*)[BM * BK]>(smem + grp * RING);
    uint8_t(*sW)[BN * BK] = reinterpret_cast<uint8_t(*)[BN * BK]>(smem + grp * RING + NSTG * BM * BK);
    float(*sS)[256] = reinterpret_cast<float(*)[256]>(smem + KSP * RING);  // GRP: [stage][tile row]
    int tm, tn;
    tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // this group's stages [kt0, kt0 + KT); every group runs KTg iterations (the barriers are workgroup-wide), the
    // ones past its own stages issue and compute nothing
    const int KTall = (K + BK - 1) / BK, KTg = (KTall + KSP - 1) / KSP;
    const int kt0 = grp * KTg, KT = max(0, min(KTall, kt0 + KTg) - kt0);

    // this lane's share of the direct loads: instruction j of wavefront w covers tile rows 16 (4 j + w) + lane / 4
    const v4i rx = make_desc(X + (size_t)m0 * K, (uint32_t)std::min<long>((long)(M - m0) * K, 0x7fffffffL));
    const v4i rw = make_desc(W + (size_t)n0 * K, (uint32_t)std::min<long>((long)(N - n0) * K, 0x7fffffffL));
    const v4i rs = make_desc(GRP ? (const void *)sx : (const void *)W, GRP ? (uint32_t)std::min<long>((long)(K / 64) * M * 4, 0x7fffffffL) : 0u);
    uint32_t ox[IX], ow[IW];
    int cx[IX], cw[IW];  // byte offset of the fetched chunk within the 64-byte row slice of a stage
#pragma unroll
    for (int j = 0; j < IX; ++j) {
        const int row = 16 * (4 * j + wave) + (lane >> 2);
        cx[j] = 16 * ((lane & 3) ^ ((row >> sh) & 3));
        ox[j] = (uint32_t)row * K + cx[j];
    }
#pragma unroll
    for (int j = 0; j < IW; ++j) {
        const int row = 16 * (4 * j + wave) + (lane >> 2);
        cw[j] = 16 * ((lane & 3) ^ ((row >> sh) & 3));
        ow[j] = (uint32_t)row * K + cw[j];
    }
    // XBF: instruction j of wavefront w loads tile rows 8 (4 j + w) .. + 7 of the stage into its bf16 slot (1 KiB,
    // 128 bytes a row); lane i takes row 8 (4 j + w) + i / 8 and its values e8 = i % 8 (8 bf16), which become int8
    // bytes 8 e8 .. + 7 of the row's 64-byte slice: logical chunk e8 / 2, half e8 % 2, at that chunk's swizzled
    // slot. Rows past M and values past K read zeros.
    uint8_t(*sXb)[BM * 2 * BK] = reinterpret_cast<uint8_t(*)[BM * 2 * BK]>(smem + KSP * RING + (GRP ? NSTG * 1024 : 0));
    v4i rxb = {};
    uint32_t oxb[IXB];
    int dxb[IXB], exb[IXB];
    float sxb[IXB], rxb_[IXB];
    if constexpr (XBF) {
        const uint16_t *Xb = reinterpret_cast<const uint16_t *>(X);
        rxb = make_desc(Xb + (size_t)m0 * K, (uint32_t)std::min<long>((long)(M - m0) * K * 2, 0x7fffffffL));
#pragma unroll
        for (int j = 0; j < IXB; ++j) {
            const int row = 8 * (4 * j + wave) + (lane >> 3), e8 = lane & 7;
            exb[j] = 8 * e8;
            oxb[j] = (uint32_t)row * K * 2 + 16 * e8;
            dxb[j] = swz(row, e8 >> 1, sh) + 8 * (e8 & 1);
            sxb[j] = m0 + row < M ? sx[m0 + row] : 1.f;
            rxb_[j] = 1.f / sxb[j];
        }
    }
    // XBF: this wavefront's rows of stage kt, bf16 slot -> int8 slot (its own direct loads of the stage have
    // landed: the caller waited; nothing else reads the bf16 slot)
    auto quant_xb = [&](int kt) {
        // the s_waitcnt builtin is not a memory operation to the compiler: keep the slot's reads below it
        asm volatile("" ::: "memory");
        const uint8_t *b_s = sXb[kt % NSTG];
        uint8_t *x_s = sX[kt % NSTG];
#pragma unroll
        for (int j = 0; j < IXB; ++j) {
            const v4i v = *reinterpret_cast<const v4i *>(b_s + 1024 * (4 * j + wave) + 16 * lane);
            int lo, hi;
            quant8(v, sxb[j], rxb_[j], lo, hi);
            *reinterpret_cast<int2 *>(x_s + dxb[j]) = make_int2(lo, hi);
        }
    };
    auto issue_in = [&](int kt, int buf) {  // kt: this group's stage index, buf = kt % NSTG
        const int k0 = (kt0 + kt) * BK;
        if constexpr (XBF)
#pragma unroll
            for (int j = 0; j < IXB; ++j) {
                const uint32_t vo = k0 + exb[j] < K ? oxb[j] + 2 * k0 : 0xfffffff0u;
                lds_dma16(rxb, vo, lds_addr(sXb[buf] + 1024 * (4 * j + wave)));
            }
        else
#pragma unroll
            for (int j = 0; j < IX; ++j) {
                // grouped scales need K % 64 == 0, so each of a stage's chunks is inside its row there
                const uint32_t vo = GRP || k0 + cx[j] < K ? ox[j] + k0 : 0xfffffff0u;
                lds_dma16(rx, vo, lds_addr(sX[buf] + 1024 * (4 * j + wave)));
            }
#pragma unroll
        for (int j = 0; j < IW; ++j) {
            const uint32_t vo = GRP || k0 + cw[j] < K ? ow[j] + k0 : 0xfffffff0u;
            lds_dma16(rw, vo, lds_addr(sW[buf] + 1024 * (4 * j + wave)));
        }
        if (GRP)  // scales sxT[kt, m0 + 64 wave + lane] (rows past the tile are loaded and not used)
            lds_dma4(rs, (uint32_t)(((long)(kt0 + kt) * M + m0 + 64 * wave + lane) * 4),
                     lds_addr(reinterpret_cast<uint8_t *>(sS[buf]) + 256 * wave));
    };
    auto issue = [&](int kt) { issue_in(kt, kt % NSTG); };

    v16f facc[GRP ? TN : 1][GRP ? TM : 1];
    if (GRP)
#pragma unroll
        for (int i = 0; i < (GRP ? TN : 1); ++i)
#pragma unroll
            for (int j = 0; j < (GRP ? TM : 1); ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) facc[i][j][e] = 0.f;

    v16i acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    const int lr = lane & 31, lh = lane >> 5;  // MFMA operand row / k-half of this lane
    int fw[2][TN], fx[2][TM];                    // fragment byte offsets within a stage buffer
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
        for (int i = 0; i < TN; ++i) fw[kk][i] = swz(wn * WNt + 32 * i + lr, 2 * kk + lh, sh);
#pragma unroll
        for (int j = 0; j < TM; ++j) fx[kk][j] = swz(wm * WMt + 32 * j + lr, 2 * kk + lh, sh);
    }

    // the MFMAs of stage kt (its operands are in LDS and visible); slot = kt % NSTG, a compile-time constant where
    // the caller knows it (the LDS addresses then fold into the reads' immediate offsets)
    auto compute_in = [&](int slot) {
        const uint8_t *x_s = sX[slot], *w_s = sW[slot];
        // both k steps' fragments are read up front, the second set while the first set's MFMAs run
        v4i wf[2][TN], xf[2][TM];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int i = 0; i < TN; ++i) wf[kk][i] = *reinterpret_cast<const v4i *>(w_s + fw[kk][i]);
#pragma unroll
            for (int j = 0; j < TM; ++j) xf[kk][j] = *reinterpret_cast<const v4i *>(x_s + fx[kk][j]);
        }
        __builtin_amdgcn_sched_barrier(0);
        const v16i zero = {};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[kk][i], xf[kk][j],
                                                                     (GRP && kk == 0) ? zero : acc[i][j], 0, 0, 0);
        if (GRP) {
            const float *s_s = sS[slot];
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const float sj = s_s[wm * WMt + 32 * j + lr];
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        facc[GRP ? i : 0][GRP ? j : 0][e] =
                            __builtin_fmaf((float)acc[i][j][e], sj, facc[GRP ? i : 0][GRP ? j : 0][e]);
            }
        }
    };

    auto compute = [&](int kt) { compute_in(kt % NSTG); };

    if constexpr (XBF) {
        // Stage kt + 2 is issued after stage kt's barrier; after stage kt's MFMAs each wavefront waits for its own
        // loads of stage kt + 1 and quantizes its activation rows into stage kt + 1's int8 slot (last read in stage
        // kt - 2), which stage kt + 1's barrier then makes visible together with its weights.
        constexpr int PER = IXB + IW;
        static_assert(PER <= 63, "vmcnt holds at most 63 loads");
        if (0 < KT) issue(0);
        if (1 < KT) issue(1);
        if (0 < KT) {
            wait_stages<PER>(1 < KT ? 1 : 0);
            quant_xb(0);
        }
        for (int kt = 0; kt < KT; ++kt) {
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (kt + 2 < KT) issue(kt + 2);
            compute(kt);
            if (kt + 1 < KT) {
                wait_stages<PER>(kt + 2 < KT ? 1 : 0);
                quant_xb(kt + 1);
            }
        }
    } else {
    static_assert((NSTG - 2) * (IX + IW + IS) <= 63 && NSTG - 2 <= 6, "vmcnt holds at most 63 loads");
#pragma unroll
    for (int p = 0; p < NSTG - 1; ++p)
        if (p < KT) issue(p);
    if constexpr (GRP && KSP == 1) {
        // the grouped fold is VALU-bound: the stage loop is unrolled by the ring depth so that each copy's slot is a
        // constant and no per-stage address arithmetic remains beside the fold (same loads, order and results).
        // With two or more tiles per wavefront the tiles form two halves and the fold is software-pipelined against
        // the matrix cores: stage kt runs half 0's MFMAs beside the fold of half 1's stage kt - 1 sums, then half 1's
        // MFMAs beside the fold of half 0's stage kt sums, each MFMA followed by its share of the fold so that the
        // SIMD runs both at once. Every accumulator is still folded once per stage, in stage order (half 1's last
        // stage after the loop; its stage -1 fold adds 0 x 0 to the zero accumulators), so the results are the
        // unpipelined ones bit for bit. No extra accumulators: half 1's stage kt - 1 sums are read before its stage
        // kt MFMAs overwrite them.
        constexpr bool PIPE = TN * TM >= 2;
        constexpr int NT = TN * TM / 2;  // tiles per half
        constexpr int VPM = 16;          // a tile's fold (16 conversions + 16 FMAs) per its two MFMAs
        auto in_half = [](int h, int i, int j) { return (TN >= 2 ? i < TN / 2 : j < TM / 2) == (h == 0); };
        float sc_prev[TM];
#pragma unroll
        for (int j = 0; j < TM; ++j) sc_prev[j] = 0.f;
        auto mfma_half = [&](int h, const v4i (&wf)[2][TN], const v4i (&xf)[2][TM]) {
            const v16i zero = {};
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
                        if (in_half(h, i, j))
                            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[kk][i], xf[kk][j], kk == 0 ? zero : acc[i][j],
                                                                             0, 0, 0);
        };
        auto fold_half = [&](int h, const float (&sc)[TM]) {
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int i = 0; i < TN; ++i)
                    if (in_half(h, i, j))
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            facc[GRP ? i : 0][GRP ? j : 0][e] =
                                __builtin_fmaf((float)acc[i][j][e], sc[j], facc[GRP ? i : 0][GRP ? j : 0][e]);
        };
        // MFMA, then VPM fold instructions, 2 NT times: the pattern the scheduler keeps for one half's MFMAs and the
        // other half's fold
        auto interleave = [&]() {
#pragma unroll
            for (int r = 0; r < 2 * NT; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
            }
        };
        // SEQ: tile t (i = t / TM, j = t % TM) accumulates its stage sum in buffer t % 2, and the previous tile's sum
        // (the previous stage's last tile for t = 0) is folded from the other buffer right after; the last tile's
        // fold therefore runs beside the next stage's first MFMAs, and each accumulator is still folded once per
        // stage in stage order (the stage -1 fold adds 0 x 0), bit-identical to the other forms
        constexpr int NTS = TN * TM;
        v16i ab[2] = {};
        float sc_last = 0.f;
        auto fold_buf = [&](int t, int buf, float sc) {
            const int i = t / TM, j = t % TM;
#pragma unroll
            for (int e = 0; e < 16; ++e)
                facc[GRP ? i : 0][GRP ? j : 0][e] = __builtin_fmaf((float)ab[buf][e], sc, facc[GRP ? i : 0][GRP ? j : 0][e]);
            // pinned here: sunk past the next tile's MFMAs, the fold would keep more than two tiles' sums alive
#pragma unroll
            for (int e = 0; e < 16; ++e) asm volatile("" : "+v"(facc[GRP ? i : 0][GRP ? j : 0][e]));
        };
        auto step = [&](int kt, auto slot_c) {
            constexpr int SLOT = decltype(slot_c)::value;
            wait_stages<IX + IW + IS>(min(NSTG - 2, KT - 1 - kt));
            // every LDS read of the previous stage completes before the barrier: the loads issued right after it
            // refill that stage's slot, and a direct-to-LDS write is not ordered after an LDS read issued earlier.
            // (With one 32 x 32 block per wavefront the compiler sinks a stage's fold, and the wait for its scale
            // read, below the next barrier; under load the refill then overtook the read.)
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (kt + NSTG - 1 < KT) issue_in(kt + NSTG - 1, (SLOT + NSTG - 1) % NSTG);
            if constexpr (SEQ) {
                const uint8_t *x_s = sX[SLOT], *w_s = sW[SLOT];
                v4i wf[2][TN], xf[2][TM];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
                    for (int i = 0; i < TN; ++i) wf[kk][i] = *reinterpret_cast<const v4i *>(w_s + fw[kk][i]);
#pragma unroll
                    for (int j = 0; j < TM; ++j) xf[kk][j] = *reinterpret_cast<const v4i *>(x_s + fx[kk][j]);
                }
                float sc[TM];
#pragma unroll
                for (int j = 0; j < TM; ++j) sc[j] = sS[SLOT][wm * WMt + 32 * j + lr];
                __builtin_amdgcn_sched_barrier(0);
                const v16i zero = {};
#pragma unroll
                for (int t = 0; t < NTS; ++t) {
                    const int i = t / TM, j = t % TM, buf = t & 1;
                    ab[buf] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[0][i], xf[0][j], zero, 0, 0, 0);
                    ab[buf] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[1][i], xf[1][j], ab[buf], 0, 0, 0);
                    if (t == 0)
                        fold_buf(NTS - 1, 1, sc_last);  // the previous stage's last tile
                    else
                        fold_buf(t - 1, buf ^ 1, sc[(t - 1) % TM]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                sc_last = sc[(NTS - 1) % TM];
            } else if constexpr (!PIPE) {
                compute_in(SLOT);
            } else {
                const uint8_t *x_s = sX[SLOT], *w_s = sW[SLOT];
                v4i wf[2][TN], xf[2][TM];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
                    for (int i = 0; i < TN; ++i) wf[kk][i] = *reinterpret_cast<const v4i *>(w_s + fw[kk][i]);
#pragma unroll
                    for (int j = 0; j < TM; ++j) xf[kk][j] = *reinterpret_cast<const v4i *>(x_s + fx[kk][j]);
                }
                float sc[TM];
#pragma unroll
                for (int j = 0; j < TM; ++j) sc[j] = sS[SLOT][wm * WMt + 32 * j + lr];
                __builtin_amdgcn_sched_barrier(0);
                mfma_half(0, wf, xf);
                fold_half(1, sc_prev);
                interleave();
                __builtin_amdgcn_sched_barrier(0);
                mfma_half(1, wf, xf);
                fold_half(0, sc);
                interleave();
                __builtin_amdgcn_sched_barrier(0);
                // the folds stay in their stage: sunk into a later one, they would keep that stage's int32 sums
                // alive beside the next stage's (registers the kernel does not have)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
#pragma unroll
                        for (int e = 0; e < 16; ++e) asm volatile("" : "+v"(facc[GRP ? i : 0][GRP ? j : 0][e]));
#pragma unroll
                for (int j = 0; j < TM; ++j) sc_prev[j] = sc[j];
            }
        };
        int kt = 0;
        for (; kt + NSTG <= KT; kt += NSTG) slot_steps<0, NSTG>(kt, step);
        slot_steps_below<0, NSTG - 1>(kt, KT, step);
        if constexpr (SEQ)
            fold_buf(NTS - 1, 1, sc_last);  // the last stage's last tile
        else if constexpr (PIPE)
            fold_half(1, sc_prev);  // half 1's last stage
    } else
    for (int kt = 0; kt < (KSP == 1 ? KT : KTg); ++kt) {
        // stage kt has landed once at most the loads of the (up to NSTG - 2) stages issued after it are outstanding
        wait_stages<IX + IW + IS>(min(NSTG - 2, KT - 1 - kt));
        // stage kt visible to all; everyone is done with stage kt - 1, whose buffer refills next. A bare s_barrier:
        // __syncthreads()' fences would make the compiler drain every outstanding load here, the prefetches included
        // (LDS needs no cache maintenance between the wavefronts of a workgroup).
        asm volatile("s_barrier" ::: "memory");
        if (KSP > 1 && kt >= KT) continue;  // this group's stages are done; it keeps meeting the barriers
        if (kt + NSTG - 1 < KT) issue(kt + NSTG - 1);
        compute(kt);
    }
    }

    __syncthreads();  // every wavefront is done with the operand ring, which now holds the epilogue slices
    if constexpr (KSP > 1) {
        // groups 1.. store their accumulators (16-byte pieces, lane-contiguous), group 0 adds them in group order
        v4i *part = reinterpret_cast<v4i *>(smem);
        auto slot = [&](int g, int i, int j, int q) { return (((((g - 1) * 4 + wave) * TN + i) * TM + j) * 4 + q) * 64 + lane; };
        if (grp > 0)
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        part[slot(grp, i, j, q)] =
                            v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        __syncthreads();
        if (grp == 0)
#pragma unroll
            for (int g = 1; g < KSP; ++g)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const v4i v = part[slot(g, i, j, q)];
#pragma unroll
                            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
                        }
        __syncthreads();  // the partials are read before group 0's epilogue slices overwrite them
        if (grp > 0) return;
    }
    if constexpr (GRP)
        epilogue<TM, TN, OUT>(facc, nullptr, sw, bias, Y, YsT, M, N, m0 + wm * WMt, n0 + wn * WNt, lane,
                              smem + wave * stage_bytes<TN>());
    else
        epilogue<TM, TN, OUT>(acc, sx, sw, bias, Y, YsT, M, N, m0 + wm * WMt, n0 + wn * WNt, lane,
                              smem + wave * stage_bytes<TN>());
}

// LDS byte offset of 16-byte chunk c of a CPR-chunk row r: chunk c is stored at slot c ^ ((r / (8 / CPR * 2)) % CPR), so
// the 16 rows a 16-lane phase of ds_read_b128 reads at one logical chunk hit 16 distinct bank groups (64 banks)
template <int CPR>
__device__ __forceinline__ int swzb(int r, int c) {
    constexpr int SH = CPR == 8 ? 1 : 2;
    return (r * CPR + (c ^ ((r >> SH) & (CPR - 1)))) * 16;
}

// ------------------------------------------------------------------------------------------------ W8A16
// y[m, n] = bf16( gelu?( acc * sw[n] + b[n] ) ), acc = sum_k x[m, k] w[n, k] in fp32 on the bf16 matrix cores
// (v_mfma_f32_32x32x16_bf16), the int8 weights converted to bf16 exactly in registers after their LDS read. Same
// workgroup shape, XCD tile order, direct-to-LDS staging and staged epilogue as the W8A8 kernel; a stage is 64 k:
// 128-byte activation rows (chunk c of row r at slot c ^ ((r >> 1) & 7)) and 64-byte weight rows (the W8A8 layout).

// 8 int8 weights (two dwords) -> 8 bf16, exact (|q| <= 128 fits the 8-bit bf16 significand): the upper halves of the
// fp32 conversions, paired by v_perm_b32
__device__ __forceinline__ v8bf w8x8_to_bf16(uint32_t d0, uint32_t d1) {
    auto hi2 = [](float lo, float hi) {
        return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
    };
    v4u r;
    r[0] = hi2((float)(int8_t)d0, (float)(int8_t)(d0 >> 8));
    r[1] = hi2((float)(int8_t)(d0 >> 16), (float)((int)d0 >> 24));
    r[2] = hi2((float)(int8_t)d1, (float)(int8_t)(d1 >> 8));
    r[3] = hi2((float)(int8_t)(d1 >> 16), (float)((int)d1 >> 24));
    return __builtin_bit_cast(v8bf, r);
}

// SPL: K is also cut into SK slices over workgroups (workgroup SK t + s takes slice s of tile t); after its own
// groups are summed, a slice's workgroup stores its fp32 accumulator registers to the workspace (register r of
// thread i at word (unit NREG + r) 256 + i), waits for them and adds one to the tile's arrival counter; the one that
// sees SK - 1 earlier arrivals sums the SK slices' registers in slice order (its own reloaded, so the order does
// not depend on which workgroup came last), resets the counter and runs the epilogue. Nothing waits.
template <int BM, int BN, int OUT, int KSP = 1, bool SPL = false>
__global__ __launch_bounds__(GT * KSP) __attribute__((amdgpu_waves_per_eu(2))) void gemm_w8_kernel(
    const uint16_t *__restrict__ X, const int8_t *__restrict__ W, const float *__restrict__ sw,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ Y, int M, int N, int K, uint32_t *__restrict__ ws = nullptr,
    int SK = 1) {
    constexpr int BKE = 64;                       // k per stage
    constexpr int WMt = BM / 2, WNt = BN / 2, TM = WMt / 32, TN = WNt / 32;
    constexpr int IX = BM / 32, IW = BN / 64;     // direct loads per wavefront per stage: X 8 rows, W 16 rows each
    constexpr int XS = BM * 2 * BKE, WS = BN * BKE;
    static_assert(IX >= 1 && IW >= 1 && TM >= 1 && TN >= 1, "tile too small");
    static_assert(4 * stage_bytes<TN>() <= STAGES * (XS + WS), "epilogue staging exceeds the LDS ring");
    // KSP > 1: KSP groups of 4 wavefronts split the K stages, each with its own ring; the fp32 partial tiles of
    // groups 1.. are added into group 0's through LDS, in group order, before the epilogue
    static_assert(KSP == 1 || (KSP - 1) * BM * BN * 4 <= KSP * STAGES * (XS + WS), "partials exceed the rings");
    constexpr int RING = STAGES * (XS + WS);
    __shared__ __attribute__((aligned(1024))) uint8_t smem[KSP * RING];

    const int tid = threadIdx.x, lane = tid & 63;
    const int grp = KSP == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid >> 8);
    const int wave = (tid >> 6) & 3;
    const int wm = wave >> 1, wn = wave & 1;
    uint8_t(*sX)[XS] = reinterpret_cast<uint8_t(*)[XS]>(smem + grp * RING);
    uint8_t(*sW)[WS] = reinterpret_cast<uint8_t(*)[WS]>(smem + grp * RING + STAGES * XS);
    int tm, tn;
    const int unit = blockIdx.x, tile = SPL ? unit / SK : unit;
    tile_of(tile, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // the workgroup's stages s0 .. s0 + SKT - 1 (all of K without SPL), split over its KSP groups
    const int KTall = (K + BKE - 1) / BKE, SPS = SPL ? (KTall + SK - 1) / SK : KTall;
    const int s0 = SPL ? (unit % SK) * SPS : 0, SKT = max(0, min(KTall, s0 + SPS) - s0);
    const int KTg = (SKT + KSP - 1) / KSP;
    const int kt0 = s0 + grp * KTg, KT = max(0, min(s0 + SKT, kt0 + KTg) - kt0);  // this group's stages kt0 .. + KT - 1
    const v4i rx = make_desc(X + (size_t)m0 * K, (uint32_t)std::min<long>((long)(M - m0) * K * 2, 0x7fffffffL));
    const v4i rw = make_desc(W + (size_t)n0 * K, (uint32_t)std::min<long>((long)(N - n0) * K, 0x7fffffffL));
    // X: instruction j of wavefront w fills rows 8 (4 j + w) .. + 7; lane i -> row + i / 8, slot i % 8
    uint32_t ox[IX], ow[IW];
    int cx[IX], cw[IW];
#pragma unroll
    for (int j = 0; j < IX; ++j) {
        const int row = 8 * (4 * j + wave) + (lane >> 3);
        cx[j] = swzb<8>(row, lane & 7) - row * 128;  // byte offset of the logical chunk stored in this slot
        ox[j] = (uint32_t)row * K * 2 + cx[j];
    }
#pragma unroll
    for (int j = 0; j < IW; ++j) {
        const int row = 16 * (4 * j + wave) + (lane >> 2);
        cw[j] = 16 * ((lane & 3) ^ ((row >> 2) & 3));
        ow[j] = (uint32_t)row * K + cw[j];
    }
    auto issue = [&](int kt) {  // kt: this group's stage index
        const int buf = kt % STAGES, k0 = (kt0 + kt) * BKE;
#pragma unroll
        for (int j = 0; j < IX; ++j) {
            const uint32_t vo = 2 * k0 + cx[j] < 2 * K ? ox[j] + 2 * k0 : 0xfffffff0u;
            lds_dma16(rx, vo, lds_addr(sX[buf] + 1024 * (4 * j + wave)));
        }
#pragma unroll
        for (int j = 0; j < IW; ++j) {
            const uint32_t vo = k0 + cw[j] < K ? ow[j] + k0 : 0xfffffff0u;
            lds_dma16(rw, vo, lds_addr(sW[buf] + 1024 * (4 * j + wave)));
        }
    };

    v16f acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int lr = lane & 31, lh = lane >> 5;

    if (KT > 0) issue(0);
    if (KT > 1) issue(1);
    for (int kt = 0; kt < (KSP == 1 ? KT : KTg); ++kt) {
        if (kt + 1 < KT)
            __builtin_amdgcn_s_waitcnt(0x3f70 | (IX + IW));
        else
            __builtin_amdgcn_s_waitcnt(0x3f70);
        asm volatile("s_barrier" ::: "memory");
        if (KSP > 1 && kt >= KT) continue;  // this group's stages are done; it keeps meeting the barriers
        if (kt + 2 < KT) issue(kt + 2);
        const uint8_t *x_s = sX[kt % STAGES], *w_s = sW[kt % STAGES];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {  // k 16 ks .. 16 ks + 15; this lane's k-half 8 lh .. 8 lh + 7
            v8bf wf[TN], xf[TM];
#pragma unroll
            for (int i = 0; i < TN; ++i) {
                const uint2 d = *reinterpret_cast<const uint2 *>(w_s + swz(wn * WNt + 32 * i + lr, ks, 2) + 8 * lh);
                wf[i] = w8x8_to_bf16(d.x, d.y);
            }
#pragma unroll
            for (int j = 0; j < TM; ++j)
                xf[j] = *reinterpret_cast<const v8bf *>(x_s + swzb<8>(wm * WMt + 32 * j + lr, 2 * ks + lh));
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();  // every wavefront is done with the operand ring, which now holds the epilogue slices
    if constexpr (KSP > 1) {
        v4f *part = reinterpret_cast<v4f *>(smem);
        auto slot = [&](int g, int i, int j, int q) { return (((((g - 1) * 4 + wave) * TN + i) * TM + j) * 4 + q) * 64 + lane; };
        if (grp > 0)
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        part[slot(grp, i, j, q)] =
                            v4f{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        __syncthreads();
        if (grp == 0)
#pragma unroll
            for (int g = 1; g < KSP; ++g)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const v4f v = part[slot(g, i, j, q)];
#pragma unroll
                            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
                        }
        __syncthreads();  // the partials are read before group 0's epilogue slices overwrite them
        if (grp > 0) return;
    }
    if constexpr (SPL) {
        constexpr int NREG = TN * TM * 16;
        constexpr int SC1 = 16;  // buffer cache policy: device-scope coherent
        const rsrc_t pr = make_rsrc(ws + SPLIT_CNT_WORDS, 0x7ffffff0u);
        auto word = [&](int u, int r) { return (uint32_t)(((u * NREG + r) * 256 + (tid & 255)) * 4); };
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][e]), pr, (int)word(unit, (i * TM + j) * 16 + e), 0, SC1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores have completed
        __shared__ uint32_t arrived;
        __syncthreads();
        if (tid == 0) arrived = __hip_atomic_fetch_add(ws + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrived != (uint32_t)(SK - 1)) return;  // uniform over the workgroup
        for (int s2 = 0; s2 < SK; ++s2) {
            float v[NREG];
#pragma unroll
            for (int r = 0; r < NREG; ++r)
                v[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, (int)word(tile * SK + s2, r), 0, SC1));
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[i][j][e] = s2 == 0 ? v[(i * TM + j) * 16 + e] : acc[i][j][e] + v[(i * TM + j) * 16 + e];
        }
        if (tid == 0) __hip_atomic_store(ws + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    epilogue<TM, TN, OUT>(acc, nullptr, sw, bias, Y, nullptr, M, N, m0 + wm * WMt, n0 + wn * WNt, lane,
                          smem + wave * stage_bytes<TN>());
}

// ------------------------------------------------------------------------------------------------ big tiles
// 256 x 256 tiles for the large GEMMs: 512 threads (8 wavefronts as 4 token blocks x 2 weight blocks, each 64 tokens x
// 128 weight rows = 2 x 4 MFMA tiles, two wavefronts per SIMD; one wavefront per SIMD with 128 x 128 blocks, which
// reads a third less LDS per MFMA, measured 10-25 % slower on every LFM2 / SigLIP2 shape). Per MAC this moves 2/3 of
// the L2 -> LDS operand bytes of the 128 x 256 kernel, which is what bounds the large shapes (the L2 runs near
// saturation there). K advances in BKT-byte stages through an NST-deep LDS ring filled by direct loads (NST - 1
// stages in flight).
// LDS rows are BKT bytes = CPR 16-byte chunks; chunk c of row r sits at slot c ^ ((r / (8 / CPR * 2)) % CPR), so
// the 16 rows a 16-lane phase of ds_read_b128 reads at one logical chunk hit 16 distinct 16-byte bank groups of the
// 64-bank LDS.

template <int OUT, int BKT, int NST>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_i8_big_kernel(
    const int8_t *__restrict__ X, const int8_t *__restrict__ W, const float *__restrict__ sx,
    const float *__restrict__ sw, const uint16_t *__restrict__ bias, void *__restrict__ Y, int M, int N, int K) {
    constexpr int WV = 8;
    constexpr int BM = 256, BN = 256, WMt = 64, WNt = 128, TM = 2, TN = 4;
    constexpr int CPR = BKT / 16;        // 16-byte chunks per LDS row
    constexpr int RPI = 64 / CPR;        // rows one direct-load instruction fills (1 KiB)
    constexpr int IL = BM / RPI / WV;    // direct-load instructions per wavefront per operand per stage
    constexpr int KS = BKT / 32;         // 32-byte MFMA k steps per stage
    static_assert(2 * NST * BM * BKT <= 160 * 1024, "LDS ring too large");
    static_assert(WV * stage_bytes<TN>() <= 2 * NST * BM * BKT, "epilogue staging exceeds the LDS ring");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * NST * BM * BKT];
    uint8_t(*sX)[BM * BKT] = reinterpret_cast<uint8_t(*)[BM * BKT]>(smem);
    uint8_t(*sW)[BN * BKT] = reinterpret_cast<uint8_t(*)[BN * BKT]>(smem + NST * BM * BKT);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = (K + BKT - 1) / BKT;

    const v4i rx = make_desc(X + (size_t)m0 * K, (uint32_t)std::min<long>((long)(M - m0) * K, 0x7fffffffL));
    const v4i rw = make_desc(W + (size_t)n0 * K, (uint32_t)std::min<long>((long)(N - n0) * K, 0x7fffffffL));
    // instruction j of wavefront w fills LDS rows RPI (WV j + w) .. + RPI - 1; lane i -> row + i / CPR, slot i % CPR
    uint32_t off[IL];
    int cb[IL];
#pragma unroll
    for (int j = 0; j < IL; ++j) {
        const int row = RPI * (WV * j + wave) + lane / CPR;
        cb[j] = swzb<CPR>(row, lane % CPR) - row * BKT;  // byte offset of the logical chunk stored in this slot
        off[j] = (uint32_t)row * K + cb[j];
    }
    auto issue = [&](int kt) {
        const int buf = kt % NST, k0 = kt * BKT;
#pragma unroll
        for (int j = 0; j < IL; ++j) {
            const bool in = k0 + cb[j] < K;
            lds_dma16(rx, in ? off[j] + k0 : 0xfffffff0u, lds_addr(sX[buf] + 1024 * (WV * j + wave)));
            lds_dma16(rw, in ? off[j] + k0 : 0xfffffff0u, lds_addr(sW[buf] + 1024 * (WV * j + wave)));
        }
    };

    v16i acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
    for (int p = 0; p < NST - 1; ++p)
        if (p < KT) issue(p);
    for (int kt = 0; kt < KT; ++kt) {
        // stage kt has landed once at most the loads of the stages after it that are in flight remain outstanding
        static_assert((NST - 2) * 2 * IL < 64, "vmcnt holds 6 bits");
        if (kt + NST - 2 < KT)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * 2 * IL));
        else
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        asm volatile("s_barrier" ::: "memory");  // everyone's loads of stage kt landed; stage kt - 1 is free
        if (kt + NST - 1 < KT) issue(kt + NST - 1);
        const uint8_t *x_s = sX[kt % NST], *w_s = sW[kt % NST];
        // the fragments of k step kk + 1 are read (into the other register set) before the MFMAs of step kk issue
        v4i wf[2][TN], xf[2][TM];
        auto rd = [&](int set, int kk) {
            const int c = 2 * kk + lh;
#pragma unroll
            for (int i = 0; i < TN; ++i)
                wf[set][i] = *reinterpret_cast<const v4i *>(w_s + swzb<CPR>(wn * WNt + 32 * i + lr, c));
#pragma unroll
            for (int j = 0; j < TM; ++j)
                xf[set][j] = *reinterpret_cast<const v4i *>(x_s + swzb<CPR>(wm * WMt + 32 * j + lr, c));
        };
        rd(0, 0);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            if (kk + 1 < KS) rd((kk + 1) & 1, kk + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[kk & 1][i], xf[kk & 1][j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();  // every wavefront is done with the operand ring, which now holds the epilogue slices
    epilogue<TM, TN, OUT>(acc, sx, sw, bias, Y, nullptr, M, N, m0 + wm * WMt, n0 + wn * WNt, lane,
                          smem + wave * stage_bytes<TN>());
}

// Persistent form of the BM x BN kernels (256 x 256, 256 x 128, 128 x 128, 128 x 64; 128-byte stages in an
// NSLOT-deep LDS ring, NSLOT - 1 of them in flight; 8 wavefronts as 4 x 2 blocks of BM/4 x BN/2): one workgroup per
// CU walks the tiles w, w + grid, ... (same XCD bands as tile_of). The smaller tiles give the shapes whose 256 x 256
// tiles leave CUs idle (w2 at 4096 tokens: 128 tiles of 256 x 256, 256 of 256 x 128; at 2048 tokens 256 of
// 128 x 128; qkv at 512 tokens 192 of 128 x 64) a tile per CU, and their smaller ring slots room for deeper rings
// (the launcher uses 3 slots for 256 x 128, 4 for 128 x 128, 6 for 128 x 64). When a tile's K loop ends, the next tile's first stage and its
// epilogue operands (the 256 token scales, 256 weight scales and 256 bias values, by direct loads into a second
// small LDS buffer) are issued before the epilogue runs, so their latency hides behind the dequant and the stores,
// and the stores drain while the next tile's first stage computes: the stage-0 wait leaves exactly the wavefront's
// SST staged stores outstanding. Staged stores are buffer stores whose out-of-range lanes get an offset past the
// buffer (dropped by the range check), so every wavefront issues the same number; the staging area is the ring
// slot the last stage used, 32 rows x BN bytes per wavefront with 16-byte granule g of row r at g ^ (r % (BN / 16)).
// bf16 output only, with N % 8 == 0, 16-byte aligned Y, 4-byte aligned bias (its dword loads) and M N 2 < 2^31
// (the launcher checks): the epilogue then issues no vector memory loads, so nothing but the staged stores is
// outstanding when the next tile's first stage is waited for.
// SPL: K is also cut into SK slices, a work unit being (tile, slice) (unit = tile SK + slice); a slice's unit stores
// its int32 accumulator registers to the workspace (register r of thread i at word (unit NREG + r) 512 + i, so every
// store instruction writes 2 KiB contiguous) with device-coherent stores, waits for them, and adds one to the tile's
// arrival counter (workspace word `tile`); the unit that sees SK - 1 earlier arrivals loads the other slices'
// registers, adds them to its own (int32: exact in any order), sets the counter back to 0 and runs the epilogue.
// Nothing waits on another workgroup. The counters must be 0 when a call starts (a zero-filled workspace; every
// completed call leaves them 0).

// ------------------------------------------------------------------------------------------------ quantizing prologue
// XQ (lfm2q_gemm_i8_fq): the persistent kernel takes bf16 activations and quantizes them itself, once, before its
// tiles: per-token scales s = max(amax, 1e-8) / 127 and q = rint(x / s) by the quantizers' own code (quant8), so the
// int8 rows, the scales and therefore every output equal quant_rows followed by the GEMM bit for bit.
//   * The rows are cut into chunks of rpc rows (at most 16384 values: 4 vectors of 8 per thread of a 512-thread
//     workgroup, and no more rows than spread the chunks over every workgroup) and chunk c belongs to workgroup
//     c % G. Each workgroup quantizes its chunks (all 512 threads on one chunk, the row maxima meeting in LDS),
//     writes the int8 rows and the scales to the caller's q and sx with device-scope stores, waits for them,
//     publishes each chunk as done in a state word and adds their number to a done count.
//   * Before its first tile a workgroup waits until the count reaches the number of chunks, then reads the int8
//     rows and scales with device-scope loads (a line of q in this XCD's L2 may be from an earlier call; one
//     agent-scope acquire fence per workgroup instead, an invalidation of the XCD's L2, measured 15 us on MI355X
//     and the device-scope loads no slower than ordinary ones in the tiles). Nothing waits on a chunk's owner for long: after
//     steal_ticks of waiting (20 us by default) the waiter quantizes, and publishes, every chunk whose state is
//     still open itself (the bytes are a function of x alone, so a second writer stores what the first did; only
//     owners add to the count), so the kernel finishes whatever runs beside it and however many of its workgroups
//     are resident.
//   * States hold epoch * 4 + 2 for done, epoch = control word 0, so they never need clearing: the last workgroup
//     to leave (control word 1 counts them) zeroes the counts (words 1 and 2) and advances the epoch. A zero-filled
//     control block is a valid start; two launches on one control block at the same time race.
constexpr int XQ_CTL = 64;                                       // control words ahead of the chunk states
constexpr int XQ_CHUNK_VALS = 16384;                             // values per chunk at most
constexpr int XQ_MAX_CHUNKS = (int)(GEMM_CTL_BYTES / 4) - XQ_CTL;  // chunk states in the control block
constexpr int XQ_WAIT_US = 20;                                   // default wait before stealing, in microseconds
constexpr uint64_t XQ_TICKS_PER_US = 100;                        // s_memrealtime runs at 100 MHz
constexpr int AUX_DEV = 16;                                      // device-scope (sc1) buffer access

// Rows per chunk for K and a grid of G workgroups: as many as 16384 values hold, but no more than ceil(M / G), so
// every workgroup gets a chunk where there are rows enough. The chunk count never exceeds that of the first bound
// or G, whichever is larger.
__host__ __device__ inline int xq_rows_per_chunk(int M, int K, int G) {
    const int cap = K >= XQ_CHUNK_VALS ? 1 : XQ_CHUNK_VALS / K, spread = (M + G - 1) / G;
    return spread < cap ? (spread > 0 ? spread : 1) : cap;
}

// Chunk c is rows r0 .. r0 + R - 1, V = R K / 8 vectors of 8 values; thread t holds vectors t + 512 j, j < 4.
struct XqChunk {
    int r0, R, V;
    __device__ XqChunk(int c, int rpc, int M, int K) : r0(c * rpc), R(min(rpc, M - c * rpc)), V(R * (K >> 3)) {}
};

__device__ __forceinline__ void xq_load(const XqChunk &ch, int K, rsrc_t rxb, int tid, v4i (&v)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = tid + 512 * j;
        v[j] = idx < ch.V ? buf_ld16_nt(rxb, (uint32_t)(((size_t)ch.r0 * K + (size_t)idx * 8) * 2)) : v4i{0, 0, 0, 0};
    }
}

// Quantize a loaded chunk with all 512 threads; smem: R floats of scratch (the rows' maxima).
__device__ __forceinline__ void xq_quant(const XqChunk &ch, int K, const v4i (&v)[4], rsrc_t rxq, rsrc_t rsx,
                                         uint8_t *smem, int tid) {
    const int C8 = K >> 3, V = ch.V;
    unsigned *rmax = reinterpret_cast<unsigned *>(smem);
    for (int i = tid; i < ch.R; i += 512) rmax[i] = 0u;
    __syncthreads();
    // the rows' maxima of |x| (non-negative fp32 values order as their bit patterns): a wavefront whose 64 vectors
    // lie in one row reduces them first and sends one value, the others one per lane
    const int wbase = tid & ~63;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = tid + 512 * j, first = wbase + 512 * j, last = first + 63;
        const float m = absmax8(v[j], 0.f);
        if (last < V && first / C8 == last / C8) {  // uniform over the wavefront
            const float wm = wave_max(m);
            if ((tid & 63) == 0) atomicMax(&rmax[first / C8], __float_as_uint(wm));
        } else if (idx < V) {
            atomicMax(&rmax[idx / C8], __float_as_uint(m));
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = tid + 512 * j;
        if (idx < V) {
            const int r = idx / C8, cv = idx - r * C8;
            const float sc = scale_of(__uint_as_float(rmax[r])), rc = 1.f / sc;
            int lo, hi;
            quant8(v[j], sc, rc, lo, hi);
            __builtin_amdgcn_raw_buffer_store_b64(v2u{(uint32_t)lo, (uint32_t)hi}, rxq,
                                                  (int)(((size_t)(ch.r0 + r) * K + (size_t)cv * 8)), 0, AUX_DEV);
            if (cv == 0) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sc), rsx, (ch.r0 + r) * 4, 0, AUX_DEV);
        }
    }
    __syncthreads();  // the maxima are read before the next chunk clears them
}

// Phase 1 of an XQ launch (every thread of the workgroup); returns the epoch, for xq_leave.
__device__ __forceinline__ uint32_t xq_prologue(const uint16_t *__restrict__ Xb, int8_t *__restrict__ Xq,
                                                float *__restrict__ sx, uint32_t *__restrict__ ctl, int M, int K,
                                                uint64_t steal_ticks, uint8_t *smem, int tid) {
    __shared__ uint32_t bcast[2];
    const int G = gridDim.x, rpc = xq_rows_per_chunk(M, K, G), nch = (M + rpc - 1) / rpc;
    const rsrc_t rxb = make_rsrc(Xb, (uint32_t)((size_t)M * K * 2)), rxq = make_rsrc(Xq, (uint32_t)((size_t)M * K));
    const rsrc_t rsx = make_rsrc(sx, (uint32_t)M * 4u);
    if (tid == 0) bcast[0] = __hip_atomic_load(ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const uint32_t epoch = bcast[0], done = epoch * 4u + 2u;
    uint32_t *state = ctl + XQ_CTL;
    int own = 0;
    for (int c = blockIdx.x; c < nch; c += G, ++own) {
        v4i v[4];
        const XqChunk ch(c, rpc, M, K);
        xq_load(ch, K, rxb, tid, v);
        xq_quant(ch, K, v, rxq, rsx, smem, tid);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores have completed
    __syncthreads();
    if (tid == 0 && own) {
        for (int c = blockIdx.x; c < nch; c += G)
            __hip_atomic_store(&state[c], done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(ctl + 2, (uint32_t)own, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // every chunk done by its owner, or after steal_ticks the ones still open quantized (and published) here
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        if (tid == 0)
            bcast[1] = __hip_atomic_load(ctl + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= (uint32_t)nch;
        __syncthreads();
        if (bcast[1]) break;  // uniform
        if (__syncthreads_or(tid == 0 && __builtin_amdgcn_s_memrealtime() - t0 >= steal_ticks)) {
            for (int c = 0; c < nch; ++c) {  // in order; each chunk that is still open, by the whole workgroup
                if (tid == 0)
                    bcast[1] = __hip_atomic_load(&state[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != done;
                __syncthreads();
                if (bcast[1]) {
                    v4i v[4];
                    const XqChunk ch(c, rpc, M, K);
                    xq_load(ch, K, rxb, tid, v);
                    xq_quant(ch, K, v, rxq, rsx, smem, tid);
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    __syncthreads();
                    if (tid == 0) __hip_atomic_store(&state[c], done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __syncthreads();
            }
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // nothing of the prologue outstanding when the ring starts
    return epoch;
}

// The workgroup leaves: the last one zeroes the counts and advances the epoch (every workgroup has read them and is
// past its last state access) for the next launch on this control block.
__device__ __forceinline__ void xq_leave(uint32_t *__restrict__ ctl, uint32_t epoch, int tid) {
    __syncthreads();
    if (tid == 0) {
        const uint32_t before = __hip_atomic_fetch_add(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (before == gridDim.x - 1) {
            __hip_atomic_store(ctl + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int OUT, int BM, int BN, int NSLOT, bool SPL = false, bool XQ = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_i8_bigp_kernel(
    const int8_t *__restrict__ X, const int8_t *__restrict__ W, const float *__restrict__ sx,
    const float *__restrict__ sw, const uint16_t *__restrict__ bias, void *__restrict__ Y, int M, int N, int K,
    uint32_t *__restrict__ ws = nullptr, int SK = 1, const uint16_t *__restrict__ Xb = nullptr,
    uint32_t *__restrict__ ctl = nullptr, uint64_t steal_ticks = 0) {
    static_assert(OUT == OUT_BF16 || OUT == OUT_BF16_GELU, "bf16 output only");
    static_assert((BM == 256 && (BN == 256 || BN == 128)) || (BM == 128 && (BN == 128 || BN == 64)), "tile shape");
    constexpr int BKT = 128, WMt = BM / 4, WNt = BN / 2, TM = WMt / 32, TN = WNt / 32;
    constexpr int CPR = BKT / 16, RPI = 64 / CPR, ILX = BM / RPI / 8, ILW = BN / RPI / 8, KS = BKT / 32;
    constexpr int SLOT = (BM + BN) * BKT;          // one stage of both operands (64 / 48 KiB)
    constexpr int EOP = 4 * BM + 4 * BN + (BN >= 128 ? 2 * BN : 256);  // one tile's sx, sw, bias (bias: 128+)
    constexpr int G = WNt / 8;                     // 16-byte granules per staged output row (2 WNt bytes)
    constexpr int RPS = 64 / G;                    // staged rows per store instruction
    constexpr int SST = TM * 32 / RPS;             // staged stores per wavefront per tile
    constexpr int LPS = ILX + ILW;                 // operand loads per wavefront per stage
    static_assert(8 * 32 * 2 * WNt <= SLOT, "epilogue staging exceeds a ring slot");
    static_assert(NSLOT >= 2 && NSLOT <= 6 && NSLOT * SLOT + 2 * EOP <= 160 * 1024, "LDS ring");
    static_assert((NSLOT - 2) * LPS + SST < 64, "vmcnt holds 6 bits");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSLOT * SLOT + 2 * EOP];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int tm_n = (M + BM - 1) / BM, tn_n = (N + BN - 1) / BN, T = tm_n * tn_n * (SPL ? SK : 1);
    const int KTT = (K + BKT - 1) / BKT;                  // stages of the whole K
    const int SPS = SPL ? (KTT + SK - 1) / SK : KTT;      // stages per slice
    int t = blockIdx.x;                                   // work unit
    // XQ: X (the int8 rows) and sx are written here first, by every workgroup of the grid (which may hold more
    // workgroups than units); otherwise the launch sizes the grid to at most T
    uint32_t epoch = 0;
    if constexpr (XQ)
        epoch = xq_prologue(Xb, const_cast<int8_t *>(X), const_cast<float *>(sx), ctl, M, K, steal_ticks, smem, tid);
    if (t >= T) {  // uniform per workgroup
        if constexpr (XQ) xq_leave(ctl, epoch, tid);
        return;
    }

    uint32_t off[ILX];
    int cb[ILX];
#pragma unroll
    for (int j = 0; j < ILX; ++j) {
        const int row = RPI * (8 * j + wave) + lane / CPR;
        cb[j] = swzb<CPR>(row, lane % CPR) - row * BKT;
        off[j] = (uint32_t)row * K + cb[j];
    }
    int m0 = 0, n0 = 0, kb = 0, KT = KTT;  // the unit's tile corner and its stages kb .. kb + KT - 1
    int utile = 0, uslice = 0;              // K split: the unit's tile (its arrival counter) and K slice
    v4i rx, rw;
    auto at_tile = [&](int tt) {
        int tm, tn;
        if (SPL && (tm_n * tn_n) % 8 == 0 && gridDim.x % 8 == 0) {
            // unit tt runs on XCD tt % 8: that XCD's band of tiles (tile_of's band), each tile's SK slices in a row,
            // so the slices of a tile and the tiles sharing operand panels meet in one L2
            const int x = tt % 8, r = tt / 8;
            utile = x * (tm_n * tn_n / 8) + r / SK;
            uslice = r % SK;
            group_of(utile, tm_n, tn_n, tm, tn);
        } else {
            utile = SPL ? tt / SK : tt;
            uslice = SPL ? tt % SK : 0;
            tile_of(utile, tm_n, tn_n, tm, tn);
        }
        m0 = tm * BM;
        n0 = tn * BN;
        if (SPL) {
            kb = uslice * SPS;
            KT = max(0, min(KTT - kb, SPS));
        }
        rx = make_desc(X + (size_t)m0 * K, (uint32_t)std::min<long>((long)(M - m0) * K, 0x7fffffffL));
        rw = make_desc(W + (size_t)n0 * K, (uint32_t)std::min<long>((long)(N - n0) * K, 0x7fffffffL));
    };
    // LDS addresses as 32-bit wavefront-uniform offsets from the array's base (scalar arithmetic only)
    const uint32_t lbase = lds_addr(smem), wbase = __builtin_amdgcn_readfirstlane(wave);
    auto issue = [&](int kt, int slot) {
        const uint32_t sX = lbase + slot * SLOT, sW = sX + BM * BKT;
        const int k0 = (kb + kt) * BKT;
#pragma unroll
        for (int j = 0; j < ILX; ++j) {
            const bool in = k0 + cb[j] < K;
            if constexpr (XQ)  // written by this launch's prologue: device-scope loads
                lds_dma16_dev(rx, in ? off[j] + k0 : 0xfffffff0u, sX + 1024 * (8 * j + wbase));
            else
                lds_dma16(rx, in ? off[j] + k0 : 0xfffffff0u, sX + 1024 * (8 * j + wbase));
            if (j < ILW) lds_dma16(rw, in ? off[j] + k0 : 0xfffffff0u, sW + 1024 * (8 * j + wbase));
        }
    };
    // the tile's token scales (waves 0 .. BM / 64 - 1, 64 each), weight scales (waves 4 .. 4 + BN / 64 - 1) and bias
    // (waves 0 .. max(1, BN / 128) - 1, 128 each: a 64-column tile reads its 64 and the next tile's) into LDS: sx at
    // 0, sw at 4 BM, bias at 4 BM + 4 BN
    const v4i rsx = make_desc(sx, (uint32_t)M * 4), rsw = make_desc(sw, (uint32_t)N * 4);
    const v4i rb = make_desc(bias, bias ? (uint32_t)N * 2 : 0u);
    auto issue_eop = [&](int e) {
        const uint32_t eb = lbase + NSLOT * SLOT + e * EOP;
        // recomputed here rather than kept live across the K loop (register pressure)
        int l = lane;
        asm volatile("" : "+v"(l));
        if (wbase < 4) {
            if (wbase < BM / 64) {
                if constexpr (XQ)
                    lds_dma4_dev(rsx, (uint32_t)(m0 + 64 * wbase + l) * 4, eb + 256 * wbase);
                else
                    lds_dma4(rsx, (uint32_t)(m0 + 64 * wbase + l) * 4, eb + 256 * wbase);
            }
            if (wbase < (BN >= 128 ? BN / 128 : 1) && bias)
                lds_dma4(rb, (uint32_t)(n0 + 128 * wbase + 2 * l) * 2, eb + 4 * BM + 4 * BN + 256 * wbase);
        } else if (wbase < 4 + BN / 64) {
            lds_dma4(rsw, (uint32_t)(n0 + 64 * (wbase - 4) + l) * 4, eb + 4 * BM + 256 * (wbase - 4));
        }
    };
    const rsrc_t ry = make_rsrc(Y, (uint32_t)((size_t)M * N * 2));

    at_tile(t);
#pragma unroll
    for (int p = 0; p < NSLOT - 1; ++p)
        if (p < KT) issue(p, p);
    issue_eop(0);
    const int lr = lane & 31, lh = lane >> 5;
    int g = 0;  // ring stage counter across tiles: stage g sits in slot g % NSLOT
    for (int it = 0;; ++it) {
        v16i acc[TN][TM];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;
        for (int kt = 0; kt < KT; ++kt, ++g) {
            // stage kt has landed once at most the loads of the f stages issued after it remain outstanding (and,
            // at a tile's first stage, the previous epilogue's staged stores, issued after those loads); the next
            // tile's epilogue-operand loads sit between its stages and the stores, so the counts only wait longer
            const int f = min(NSLOT - 2, KT - 1 - kt);
            const bool st = kt == 0 && it > 0;
#define LFM2Q_WAIT_STAGE(F_)                                                                                       \
    do {                                                                                                            \
        if (st)                                                                                                     \
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((F_) * LPS + SST));                                                \
        else                                                                                                        \
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((F_) * LPS));                                                      \
    } while (0)
            if (NSLOT >= 6 && f == 4)
                LFM2Q_WAIT_STAGE(4);
            else if (NSLOT >= 5 && f == 3)
                LFM2Q_WAIT_STAGE(3);
            else if (NSLOT >= 4 && f == 2)
                LFM2Q_WAIT_STAGE(2);
            else if (NSLOT >= 3 && f == 1)
                LFM2Q_WAIT_STAGE(1);
            else
                LFM2Q_WAIT_STAGE(0);
#undef LFM2Q_WAIT_STAGE
            asm volatile("s_barrier" ::: "memory");  // every wavefront's loads of stage kt landed; slot g - 1 is free
            if (kt + NSLOT - 1 < KT) issue(kt + NSLOT - 1, (g + NSLOT - 1) % NSLOT);
            const uint8_t *x_s = smem + (g % NSLOT) * SLOT, *w_s = x_s + BM * BKT;
            v4i wf[2][TN], xf[2][TM];
            auto rd = [&](int set, int kk) {
                const int c = 2 * kk + lh;
#pragma unroll
                for (int i = 0; i < TN; ++i)
                    wf[set][i] = *reinterpret_cast<const v4i *>(w_s + swzb<CPR>(wn * WNt + 32 * i + lr, c));
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    xf[set][j] = *reinterpret_cast<const v4i *>(x_s + swzb<CPR>(wm * WMt + 32 * j + lr, c));
            };
            rd(0, 0);
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                if (kk + 1 < KS) rd((kk + 1) & 1, kk + 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[kk & 1][i], xf[kk & 1][j], acc[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // the next tile's first NSLOT - 1 stages (slots g .. g + NSLOT - 2, every slot but the last stage's: free
        // since the barrier of this tile's last stage) and epilogue operands go out before this tile's epilogue
        const int tnext = t + (int)gridDim.x;
        const int pm0 = m0, pn0 = n0, ptile = utile, pslice = uslice;
        if (tnext < T) {
            at_tile(tnext);
#pragma unroll
            for (int p = 0; p < NSLOT - 1; ++p)
                if (p < KT) issue(p, (g + p) % NSLOT);
            issue_eop((it + 1) & 1);
        }
        asm volatile("s_barrier" ::: "memory");  // every wavefront is done with the last stage's slot
        const int mb = pm0 + wm * WMt, nb = pn0 + wn * WNt;
        bool epi = true;
        if constexpr (SPL) {
            constexpr int NREG = TN * TM * 16;
            constexpr int SC1 = 16;  // buffer cache policy: device-scope coherent
            const rsrc_t pr = make_rsrc(ws + SPLIT_CNT_WORDS, 0x7ffffff0u);
            auto word = [&](int unit, int r) { return (uint32_t)(((unit * NREG + r) * 512 + tid) * 4); };
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        __builtin_amdgcn_raw_buffer_store_b32((uint32_t)acc[i][j][e], pr, (int)word(ptile * SK + pslice, (i * TM + j) * 16 + e), 0, SC1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores have completed
            __shared__ uint32_t arrived;
            __syncthreads();
            if (tid == 0) arrived = __hip_atomic_fetch_add(ws + ptile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            epi = arrived == (uint32_t)(SK - 1);  // uniform over the workgroup
            if (epi) {
                for (int s2 = 0; s2 < SK; ++s2) {
                    if (s2 == pslice) continue;
                    int v[NREG];
#pragma unroll
                    for (int r = 0; r < NREG; ++r)
                        v[r] = (int)__builtin_amdgcn_raw_buffer_load_b32(pr, (int)word(ptile * SK + s2, r), 0, SC1);
#pragma unroll
                    for (int i = 0; i < TN; ++i)
#pragma unroll
                        for (int j = 0; j < TM; ++j)
#pragma unroll
                            for (int e = 0; e < 16; ++e) acc[i][j][e] += v[(i * TM + j) * 16 + e];
                }
                if (tid == 0) __hip_atomic_store(ws + ptile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (epi) {
            const uint8_t *eb = smem + NSLOT * SLOT + (it & 1) * EOP;
            const float *sxs = reinterpret_cast<const float *>(eb);
            const float *sws = reinterpret_cast<const float *>(eb + 4 * BM);
            const uint16_t *bs = reinterpret_cast<const uint16_t *>(eb + 4 * BM + 4 * BN);
            uint8_t *stage = smem + ((g + NSLOT - 1) % NSLOT) * SLOT + wave * (32 * 2 * WNt);
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const float s_m = sxs[wm * WMt + 32 * j + lr];
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int nl = wn * WNt + 32 * i + 8 * q + 4 * lh;
                        const v4f w4 = *reinterpret_cast<const v4f *>(sws + nl);
                        uint32_t b01 = 0, b23 = 0;
                        if (bias) {
                            const uint2 bb = *reinterpret_cast<const uint2 *>(bs + nl);
                            b01 = bb.x;
                            b23 = bb.y;
                        }
                        float v[4];
                        v[0] = dequant(acc[i][j][4 * q], s_m, w4[0], bf2f_lo(b01));
                        v[1] = dequant(acc[i][j][4 * q + 1], s_m, w4[1], bf2f_hi(b01));
                        v[2] = dequant(acc[i][j][4 * q + 2], s_m, w4[2], bf2f_lo(b23));
                        v[3] = dequant(acc[i][j][4 * q + 3], s_m, w4[3], bf2f_hi(b23));
                        if (out_gelu(OUT))
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = gelu_tanh_f32(v[e]);
                        *reinterpret_cast<uint2 *>(stage + lr * (2 * WNt) + (((4 * i + q) ^ (lr & (G - 1))) << 4) +
                                                   8 * lh) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                    }
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int rr = 0; rr < 32; rr += RPS) {
                    const int r = rr + lane / G, c = lane % G;
                    const v4i v = *reinterpret_cast<const v4i *>(stage + r * (2 * WNt) + ((c ^ (r & (G - 1))) << 4));
                    const int mo = mb + 32 * j + r, no = nb + 8 * c;
                    const uint32_t o = (mo < M && no < N) ? (uint32_t)(((size_t)mo * N + no) * 2) : 0xfffffff0u;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), ry, (int)o, 0, 0);
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        if (tnext >= T) break;
        t = tnext;
    }
    if constexpr (XQ) xq_leave(ctl, epoch, tid);
}

// ------------------------------------------------------------------------------------------------ dispatch
// Tile choice by a two-term cost model fitted to MI355X timings of the seven configurations over the LFM2 prefill and
// SigLIP2 vision shapes: with `per` = ceil(tiles / CUs) tiles on the busiest CU, time ~ a x per x BM x BN x K (the
// CU's matrix-core work, a = microseconds per million MACs, lower for bigger tiles) + b x ceil(per / resident) (b =
// per-round prologue / epilogue cost, `resident` = workgroups one CU holds). The LFM2Q_GEMM_BM / _BN knobs force a tile.
struct TileCfg {
    int bm, bn, resident;
    double a, b;
    int ksp = 1;   // wavefront groups splitting K inside the workgroup (per-token path)
    int pers = 0;  // the persistent BM x BN kernel (per-token bf16 output, where its conditions hold)
    int sk = 1;    // K slices over workgroups (persistent 256 x 128 / 128 x 128 with a workspace)
};

// Tile sets: per-token (all seven), grouped (the four tiles whose fp32 accumulators fit beside the int32 ones), and
// INT8 output (grouped tiles with 64-column wavefront blocks).
enum TileSet { TILES_ALL = 0, TILES_GROUPED = 1, TILES_Q8 = 2 };

inline bool tile_in(const TileCfg &o, int set) {
    if (set == TILES_ALL) return true;
    const bool small = o.bm <= 128 && o.bn <= 128;
    return set == TILES_GROUPED ? small : small && o.bn == 128;
}

inline TileCfg pick_tile(int M, int N, int K, int set = TILES_ALL) {
    const int force_bm = knob_int(KNOB_GEMM_BM, 0), force_bn = knob_int(KNOB_GEMM_BN, 0);
    static const TileCfg opts[] = {{256, 256, 1, 0.1488, 18.64}, {128, 256, 2, 0.2726, 10.38},
                                   {256, 128, 2, 0.2795, 9.88},  {128, 128, 3, 0.3312, 4.92},
                                   {128, 64, 4, 0.4559, 1.98},   {64, 128, 4, 0.4571, 2.03},
                                   {64, 64, 6, 0.5926, 0.08}};
    if (force_bm && force_bn)
        for (const TileCfg &o : opts)
            if (o.bm == force_bm && o.bn == force_bn && tile_in(o, set)) return o;
    const long cus = device_cus();
    double best = 1e300;
    TileCfg bestc = opts[3];
    for (const TileCfg &o : opts) {
        if (!tile_in(o, set)) continue;
        const long tiles = (long)((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn);
        const long per = (tiles + cus - 1) / cus;
        const double t = o.a * (double)per * o.bm * o.bn * (double)K * 1e-6 + o.b * (double)((per + o.resident - 1) / o.resident);
        if (t < best) {
            best = t;
            bestc = o;
        }
    }
    return bestc;
}

// Per-token path: the seven tiles, each also with K split over 2 (and, for the small tiles, 4) wavefront groups,
// and the persistent 256 x 128, 128 x 128 and 128 x 64 kernels, fitted like the table above to MI355X timings of every (tile, split) on the
// 13 LFM2 prefill / SigLIP2 shapes (`resident` = workgroups one CU holds at that split). The LFM2Q_GEMM_BM / _BN
// knobs force a tile, LFM2Q_GEMM_KSPLIT its split (default 1 when a tile is forced); 256 x 128, 128 x 128 or 128 x 64
// forced means the persistent kernel unless LFM2Q_GEMM_BIGP is 0.
// With a workspace the persistent 256 x 128, 128 x 128 and 128 x 64 kernels are also candidates with K cut into SK = 2..8
// slices over workgroups (at most two units per CU, partials within the workspace), costed as their tiles on
// SK x the tiles with K / SK each plus SPLIT_US for the partial round trip; LFM2Q_GEMM_SPLITK forces SK.
constexpr double SPLIT_US = 4.0;

inline int split_fits(const TileCfg &o, long tiles, int sk, int K, size_t ws_bytes) {
    const long cus = device_cus();
    return o.pers && o.bm * o.bn <= 256 * 128 && tiles * sk <= 2 * cus && sk <= (K + 127) / 128 &&
           tiles <= (long)SPLIT_CNT_WORDS && 4 * (size_t)SPLIT_CNT_WORDS + (size_t)tiles * sk * o.bm * o.bn * 4 <= ws_bytes;
}

inline TileCfg pick_tile_pt(int M, int N, int K, size_t ws_bytes = 0, bool pers_only = false) {
    const int force_bm = knob_int(KNOB_GEMM_BM, 0), force_bn = knob_int(KNOB_GEMM_BN, 0);
    const int force_ks = pers_only ? 0 : knob_int(KNOB_GEMM_KSPLIT, 0), force_sk = knob_int(KNOB_GEMM_SPLITK, 0);
    const bool pers_ok = pers_only || knob_int(KNOB_GEMM_BIGP, 1) != 0;
    static const TileCfg opts[] = {
        {256, 256, 1, 0.1582, 10.87, 1, 1}, {256, 128, 1, 0.2033, 5.808, 1, 1}, {128, 128, 1, 0.2894, 2.859, 1, 1},
        {128, 64, 1, 0.4104, 1.750, 1, 1},
        {128, 256, 2, 0.2912, 7.604, 1}, {128, 256, 1, 0.2721, 10.14, 2},
        {256, 128, 2, 0.2911, 7.455, 1}, {256, 128, 1, 0.2572, 10.95, 2}, {128, 128, 3, 0.3494, 5.003, 1},
        {128, 128, 1, 0.3449, 5.533, 2}, {128, 64, 4, 0.4546, 3.930, 1},  {128, 64, 2, 0.4729, 2.456, 2},
        {128, 64, 1, 0.5114, 3.760, 4},  {64, 128, 4, 0.4555, 3.970, 1},  {64, 128, 2, 0.4864, 2.494, 2},
        {64, 128, 1, 0.5502, 3.505, 4},  {64, 64, 6, 0.5660, 3.086, 1},   {64, 64, 3, 0.6101, 0.836, 2},
        {64, 64, 1, 0.7027, 2.256, 4}};
    const auto usable = [&](const TileCfg &o) {
        return pers_only ? o.pers == 1 : pers_ok || !o.pers || (o.bm == 256 && o.bn == 256);
    };
    if (force_bm && force_bn) {
        const int ks = force_ks == 4 ? 4 : force_ks == 2 ? 2 : 1;
        for (const TileCfg &o : opts)
            if (o.bm == force_bm && o.bn == force_bn && o.ksp == ks && usable(o)) {
                TileCfg r = o;
                const long tiles = (long)((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn);
                if (force_sk > 1 && split_fits(o, tiles, force_sk, K, ws_bytes)) r.sk = force_sk;
                return r;
            }
        for (const TileCfg &o : opts)
            if (o.bm == force_bm && o.bn == force_bn && o.ksp == 1 && usable(o)) return o;
    }
    const long cus = device_cus();
    double best = 1e300;
    TileCfg bestc = pers_only ? opts[2] : opts[8];
    for (const TileCfg &o : opts) {
        if ((force_ks && o.ksp != force_ks) || !usable(o)) continue;
        const long tiles = (long)((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn);
        const long per = (tiles + cus - 1) / cus;
        const double t = o.a * (double)per * o.bm * o.bn * (double)K * 1e-6 + o.b * (double)((per + o.resident - 1) / o.resident);
        if (t < best) {
            best = t;
            bestc = o;
        }
        if (ws_bytes && force_sk != 1)
            for (int sk = 2; sk <= 8; ++sk) {
                if ((force_sk && sk != force_sk) || !split_fits(o, tiles, sk, K, ws_bytes)) continue;
                const long sper = (tiles * sk + cus - 1) / cus;
                const double ts = o.a * (double)sper * o.bm * o.bn * (double)((K + sk - 1) / sk) * 1e-6 +
                                  o.b * (double)sper + SPLIT_US;
                if (ts < best) {
                    best = ts;
                    bestc = o;
                    bestc.sk = sk;
                }
            }
    }
    return bestc;
}

template <int OUT>
void launch_gemm(const int8_t *A, const int8_t *B, const float *sx, const float *sw, const uint16_t *bias, void *Y,
                 int M, int N, int K, hipStream_t st, void *ws = nullptr, size_t ws_bytes = 0) {
    const TileCfg t = pick_tile_pt(M, N, K, (OUT == OUT_BF16 || OUT == OUT_BF16_GELU) && ws ? std::min(ws_bytes, GEMM_SPLIT_BYTES) : 0);
    const int sh = knob_int(KNOB_GEMM_SWZ, 2);
    const dim3 grid(((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn));
    if (t.pers) {
        if constexpr (OUT == OUT_BF16 || OUT == OUT_BF16_GELU) {
            // persistent form: one workgroup per CU (its LDS allows no second), at most one per tile
            if (knob_int(KNOB_GEMM_BIGP, 1) && K > 0 && (N & 7) == 0 && ((uintptr_t)Y & 15) == 0 &&
                ((uintptr_t)bias & 3) == 0 && (size_t)M * N * 2 < 0x80000000ull) {
                const int pgrid = (int)std::min<long>((long)grid.x, device_cus());
                // LDS ring: as many slots as LDS holds (2, 3, 4); LFM2Q_GEMM_STAGES = 2 forces two
                const bool two = knob_int(KNOB_GEMM_STAGES, 0) == 2;
                if (t.sk > 1) {
                    const int sgrid = (int)std::min<long>((long)grid.x * t.sk, device_cus());
                    uint32_t *w = static_cast<uint32_t *>(ws);
                    if (t.bm == 256)
                        gemm_i8_bigp_kernel<OUT, 256, 128, 3, true><<<sgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K,
                                                                                           w, t.sk);
                    else if (t.bn == 64)
                        gemm_i8_bigp_kernel<OUT, 128, 64, 6, true><<<sgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K,
                                                                                          w, t.sk);
                    else
                        gemm_i8_bigp_kernel<OUT, 128, 128, 4, true><<<sgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K,
                                                                                           w, t.sk);
                    return;
                }
                if (t.bm == 256 && t.bn == 256)
                    gemm_i8_bigp_kernel<OUT, 256, 256, 2><<<pgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K);
                else if (t.bm == 256 && two)
                    gemm_i8_bigp_kernel<OUT, 256, 128, 2><<<pgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K);
                else if (t.bm == 256)
                    gemm_i8_bigp_kernel<OUT, 256, 128, 3><<<pgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K);
                else if (t.bn == 64)
                    gemm_i8_bigp_kernel<OUT, 128, 64, 6><<<pgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K);
                else if (two)
                    gemm_i8_bigp_kernel<OUT, 128, 128, 2><<<pgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K);
                else
                    gemm_i8_bigp_kernel<OUT, 128, 128, 4><<<pgrid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K);
                return;
            }
        }
    }
    if (t.bm == 256 && t.bn == 256) {
        // ring shape (K bytes per stage x stages); the LFM2Q_GEMM_RING knob (1282 / 644 / 645) forces one
        switch (knob_int(KNOB_GEMM_RING, 1282)) {
        case 644: gemm_i8_big_kernel<OUT, 64, 4><<<grid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K); break;
        case 645: gemm_i8_big_kernel<OUT, 64, 5><<<grid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K); break;
        default: gemm_i8_big_kernel<OUT, 128, 2><<<grid, 512, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K); break;
        }
        return;
    }
    // LDS ring depth 6 (4 stages in flight) for a small tile whose grid leaves one workgroup per CU on a long K: a
    // lone workgroup with 2 stages in flight is bound by the operand latency (w2 at 512 tokens: 45 -> 35 us); the
    // deeper ring's LDS costs occupancy everywhere else. The LFM2Q_GEMM_STAGES knob (3 / 6) forces it (6 for any tile but
    // 256 x 256, which has its own ring).
    const bool small = t.bm + t.bn <= 192;
    int nst = (small && (long)grid.x <= device_cus() && K >= 4096) ? 6 : 3;
    if (const int f = knob_int(KNOB_GEMM_STAGES, 0)) nst = f == 6 && t.bm + t.bn <= 384 ? 6 : 3;
    // K split inside the workgroup (t.ksp groups of 4 wavefronts, int32 partials summed in LDS): where the tiles
    // leave one workgroup per CU, a lone workgroup's stage is bound by its LDS -> MFMA dependency chain and a second
    // or fourth group of wavefronts on other K stages fills the CU (w2 at 512 tokens: 36 -> 27 us).
    const int ksp = t.ksp;
    if (ksp > 1) nst = 3;
#define LFM2Q_GEMM(BM_, BN_)                                                                                        \
    if (t.bm == BM_ && t.bn == BN_) {                                                                                \
        if (ksp == 4 && BM_ + BN_ <= 192)                                                                            \
            gemm_i8_kernel<BM_, BN_, OUT, false, STAGES, (BM_ + BN_ <= 192 ? 4 : 1)><<<grid, 4 * GT, 0, st>>>(       \
                A, B, sx, sw, bias, Y, M, N, K, sh);                                                                 \
        else if (ksp == 2)                                                                                           \
            gemm_i8_kernel<BM_, BN_, OUT, false, STAGES, 2><<<grid, 2 * GT, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K, \
                                                                                      sh);                           \
        else if (BM_ + BN_ <= 384 && nst == 6)                                                                       \
            gemm_i8_kernel<BM_, BN_, OUT, false, (BM_ + BN_ <= 384 ? 6 : 3)><<<grid, GT, 0, st>>>(A, B, sx, sw,      \
                                                                                                  bias, Y, M, N, K, sh); \
        else                                                                                                         \
            gemm_i8_kernel<BM_, BN_, OUT><<<grid, GT, 0, st>>>(A, B, sx, sw, bias, Y, M, N, K, sh);                 \
        return;                                                                                                      \
    }
    LFM2Q_GEMM(128, 256)
    LFM2Q_GEMM(256, 128)
    LFM2Q_GEMM(128, 128)
    LFM2Q_GEMM(128, 64)
    LFM2Q_GEMM(64, 128)
    LFM2Q_GEMM(64, 64)
#undef LFM2Q_GEMM
}

// bf16 activations quantized by the persistent kernel's own prologue (q, sx: quant_rows' bytes), the persistent
// configurations only, every CU in the grid (a workgroup with no tile quantizes and leaves). True where the knob
// LFM2Q_GEMM_FQ = 1 asks for it and the shape and pointers fit the persistent kernel; otherwise the caller runs the
// pair (quant_rows, then the GEMM), which is the default because it is the faster form on MI355X: the prologue's
// wait for every chunk (device-scope counts seen across the XCDs) and its leaving count cost 5-10 us more than the
// kernel boundary they replace, and its chunks stream no faster than quant_rows' grid.
inline bool fq_applies(int M, int N, int K, const void *Y, const void *bias) {
    const int rpc = xq_rows_per_chunk(M, K, 1);
    return knob_int(KNOB_GEMM_FQ, 0) == 1 && K <= XQ_CHUNK_VALS && (M + rpc - 1) / rpc <= XQ_MAX_CHUNKS &&
           (N & 7) == 0 && ((uintptr_t)Y & 15) == 0 && ((uintptr_t)bias & 3) == 0 &&
           (size_t)M * N * 2 < 0x80000000ull && (size_t)M * K * 2 < 0x80000000ull;
}

template <int OUT>
void launch_gemm_fq(const uint16_t *X, int8_t *q, float *sx, const int8_t *B, const float *sw, const uint16_t *bias,
                    void *Y, int M, int N, int K, hipStream_t st, void *ws) {
    const TileCfg t = pick_tile_pt(M, N, K, GEMM_SPLIT_BYTES, true);
    const int grid = (int)device_cus();
    uint32_t *const w = static_cast<uint32_t *>(ws);
    uint32_t *const ctl = reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(ws) + GEMM_SPLIT_BYTES);
    const uint64_t ticks = (uint64_t)knob_int(KNOB_GEMM_FQ_WAIT_US, XQ_WAIT_US) * XQ_TICKS_PER_US;
#define LFM2Q_FQ(BM_, BN_, NS_, SPL_)                                                                               \
    gemm_i8_bigp_kernel<OUT, BM_, BN_, NS_, SPL_, true><<<grid, 512, 0, st>>>(q, B, sx, sw, bias, Y, M, N, K, w, t.sk,\
                                                                            X, ctl, ticks)
    if (t.sk > 1) {
        if (t.bm == 256)
            LFM2Q_FQ(256, 128, 3, true);
        else if (t.bn == 64)
            LFM2Q_FQ(128, 64, 6, true);
        else
            LFM2Q_FQ(128, 128, 4, true);
    } else if (t.bm == 256 && t.bn == 256) {
        LFM2Q_FQ(256, 256, 2, false);
    } else if (t.bm == 256) {
        LFM2Q_FQ(256, 128, 3, false);
    } else if (t.bn == 64) {
        LFM2Q_FQ(128, 64, 6, false);
    } else {
        LFM2Q_FQ(128, 128, 4, false);
    }
#undef LFM2Q_FQ
}

// grouped-64 activation scales (sxT [K/64, M]); OUT_Q8*: Y = Yq int8 [M, N], YsT [N/64, M]
template <int OUT>
void launch_gemm_grouped(const int8_t *A, const int8_t *B, const float *sxT, const float *sw, const uint16_t *bias,
                         void *Y, float *YsT, int M, int N, int K, hipStream_t st) {
    const TileCfg t = pick_tile(M, N, K, out_q8(OUT) ? TILES_Q8 : TILES_GROUPED);
    const int sh = knob_int(KNOB_GEMM_SWZ, 2);
    // a 4-stage ring (three stages in flight; 68 KiB for 128 x 128, still two workgroups a CU): equal to the
    // 3-stage ring where two workgroups share each CU, 24 % faster where the tiles leave one or none (512 x 8192 x
    // 2048); 6 stages (one workgroup a CU) were 50 % slower on the large shapes. LFM2Q_GEMM_STAGES = 3 keeps 3.
    const bool three = knob_int(KNOB_GEMM_STAGES, 0) == 3;
    const dim3 grid(((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn));
#define LFM2Q_GEMM(BM_, BN_)                                                                                        \
    if (t.bm == BM_ && t.bn == BN_) {                                                                                \
        if (three)                                                                                                   \
            gemm_i8_kernel<BM_, BN_, OUT, true, 3><<<grid, GT, 0, st>>>(A, B, sxT, sw, bias, Y, M, N, K, sh, YsT);   \
        else                                                                                                         \
            gemm_i8_kernel<BM_, BN_, OUT, true, 4><<<grid, GT, 0, st>>>(A, B, sxT, sw, bias, Y, M, N, K, sh, YsT);   \
        return;                                                                                                      \
    }
    // 128 x 128 tiles, more than two a CU: the tile-sequential fold (158 VGPRs: three wavefronts a SIMD) on a 3-stage
    // ring (51 KiB: three workgroups a CU), against two of each for the pipelined fold. Measured on MI355X: 5-7 %
    // faster from 720 tiles (4096 x 2048 x 16384 240.3 -> 224.0 us, the vision shapes 5-7 %), neutral to 3 % slower
    // at 256-512 tiles, where every tile is resident at two a CU. LFM2Q_GEMM_GSEQ = 0 / 1 forces it off / on
    // (LFM2Q_GEMM_STAGES = 3 alone keeps the pipelined fold on its 3-stage ring).
    const int gseq = knob_int(KNOB_GEMM_GSEQ, -1);
    if (t.bm == 128 && t.bn == 128 && (gseq >= 0 ? gseq == 1 : !three && (long)grid.x > 2L * device_cus())) {
        gemm_i8_kernel<128, 128, OUT, true, 3, 1, false, true><<<grid, GT, 0, st>>>(A, B, sxT, sw, bias, Y, M, N, K, sh,
                                                                                   YsT);
        return;
    }
    LFM2Q_GEMM(128, 128)
    LFM2Q_GEMM(64, 128)
    if constexpr (!out_q8(OUT)) {
        LFM2Q_GEMM(128, 64)
        LFM2Q_GEMM(64, 64)
    }
#undef LFM2Q_GEMM
}

// bf16 activations quantized inside the GEMM (sx = their quant_rows scales): the tiles of at most 128 token rows
template <int OUT>
void launch_gemm_bf16a(const uint16_t *X, const int8_t *B, const float *sx, const float *sw, const uint16_t *bias,
                       void *Y, int M, int N, int K, hipStream_t st) {
    const TileCfg t = pick_tile(M, N, K, TILES_GROUPED);
    const int sh = knob_int(KNOB_GEMM_SWZ, 2);
    const dim3 grid(((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn));
    const int8_t *Xv = reinterpret_cast<const int8_t *>(X);
#define LFM2Q_GEMM(BM_, BN_)                                                                                        \
    if (t.bm == BM_ && t.bn == BN_) {                                                                                \
        gemm_i8_kernel<BM_, BN_, OUT, false, 3, 1, true><<<grid, GT, 0, st>>>(Xv, B, sx, sw, bias, Y, M, N, K, sh);  \
        return;                                                                                                      \
    }
    LFM2Q_GEMM(128, 128)
    LFM2Q_GEMM(128, 64)
    LFM2Q_GEMM(64, 128)
    LFM2Q_GEMM(64, 64)
#undef LFM2Q_GEMM
}

template <int OUT>
void launch_gemm_w8(const uint16_t *X, const int8_t *W, const float *sw, const uint16_t *bias, uint16_t *Y, int M,
                    int N, int K, hipStream_t st, void *ws = nullptr, size_t ws_bytes = 0) {
    const TileCfg t = pick_tile(M, N, K, TILES_GROUPED);
    const long tiles = (long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
    const int KT = (K + 63) / 64;
    // With a workspace, K slices over workgroups where the tiles leave more than half the CUs idle: SK = CUs / tiles,
    // at most 8 and with at least 2048 k per slice (shorter slices lost to the unsplit kernel on MI355X: w1|w3 at 64
    // tokens 14.4 -> 15.8 us split in two, against w2 at 64 tokens 33.7 -> 15.3 us in four); LFM2Q_GEMM_SPLITK
    // forces SK (1 = none).
    int sk = 1;
    if (ws) {
        const long cus = device_cus();
        sk = (int)std::min<long>(8, std::min<long>(cus / tiles, K / 2048));
        if (const int f = knob_int(KNOB_GEMM_SPLITK, 0)) sk = std::min(f, std::max(1, KT));
        while (sk > 1 && 4 * (size_t)SPLIT_CNT_WORDS + (size_t)tiles * sk * t.bm * t.bn * 4 > std::min(ws_bytes, GEMM_SPLIT_BYTES)) --sk;
        if (tiles > (long)SPLIT_CNT_WORDS || sk < 2) sk = 1;
    }
    const dim3 grid(tiles * sk);
    // K split inside the workgroup where the tiles leave at most one workgroup per CU (a lone workgroup of 4
    // wavefronts is bound by its LDS -> convert -> MFMA chain): 4 groups for 64 x 64 tiles, 2 for the others (LDS).
    // The LFM2Q_GEMM_KSPLIT knob (1 / 2 / 4) forces it (4 only for 64 x 64).
    const bool s64 = t.bm == 64 && t.bn == 64;
    int ksp = ((long)grid.x <= device_cus() && KT / sk >= 8) ? (s64 ? 4 : 2) : 1;
    if (const int f = knob_int(KNOB_GEMM_KSPLIT, 0)) ksp = f == 4 && s64 ? 4 : f == 2 ? 2 : 1;
    uint32_t *const w = static_cast<uint32_t *>(ws);
    if (sk > 1) {
#define LFM2Q_GEMM(BM_, BN_)                                                                                        \
    if (t.bm == BM_ && t.bn == BN_) {                                                                                \
        if (ksp == 4 && BM_ == 64 && BN_ == 64)                                                                      \
            gemm_w8_kernel<BM_, BN_, OUT, (BM_ == 64 && BN_ == 64 ? 4 : 1), true><<<grid, 4 * GT, 0, st>>>(          \
                X, W, sw, bias, Y, M, N, K, w, sk);                                                                  \
        else if (ksp == 2)                                                                                           \
            gemm_w8_kernel<BM_, BN_, OUT, 2, true><<<grid, 2 * GT, 0, st>>>(X, W, sw, bias, Y, M, N, K, w, sk);     \
        else                                                                                                         \
            gemm_w8_kernel<BM_, BN_, OUT, 1, true><<<grid, GT, 0, st>>>(X, W, sw, bias, Y, M, N, K, w, sk);         \
        return;                                                                                                      \
    }
        LFM2Q_GEMM(128, 128)
        LFM2Q_GEMM(128, 64)
        LFM2Q_GEMM(64, 128)
        LFM2Q_GEMM(64, 64)
#undef LFM2Q_GEMM
    }
#define LFM2Q_GEMM(BM_, BN_)                                                                                        \
    if (t.bm == BM_ && t.bn == BN_) {                                                                                \
        if (ksp == 4 && BM_ == 64 && BN_ == 64)                                                                      \
            gemm_w8_kernel<BM_, BN_, OUT, (BM_ == 64 && BN_ == 64 ? 4 : 1)><<<grid, 4 * GT, 0, st>>>(X, W, sw, bias, \
                                                                                                  Y, M, N, K);       \
        else if (ksp == 2)                                                                                           \
            gemm_w8_kernel<BM_, BN_, OUT, 2><<<grid, 2 * GT, 0, st>>>(X, W, sw, bias, Y, M, N, K);                  \
        else                                                                                                         \
            gemm_w8_kernel<BM_, BN_, OUT><<<grid, GT, 0, st>>>(X, W, sw, bias, Y, M, N, K);                         \
        return;                                                                                                      \
    }
    LFM2Q_GEMM(128, 128)
    LFM2Q_GEMM(128, 64)
    LFM2Q_GEMM(64, 128)
    LFM2Q_GEMM(64, 64)
#undef LFM2Q_GEMM
}

int check_gemm(const char *name, const int8_t *A, const int8_t *B, const void *Y, int M, int N, int K) {
    LFM2Q_REQUIRE(A && B && Y, LFM2Q_ERR_ARG, "%s: null pointer", name);
    LFM2Q_REQUIRE(M >= 1 && N >= 1 && K >= 16, LFM2Q_ERR_SHAPE, "%s: need M, N >= 1 and K >= 16 (M=%d N=%d K=%d)",
                  name, M, N, K);
    LFM2Q_REQUIRE(K % 16 == 0, LFM2Q_ERR_SHAPE, "%s: need K %% 16 == 0 (K=%d)", name, K);
    LFM2Q_REQUIRE((long)M * K < (1L << 31) && (long)N * K < (1L << 31), LFM2Q_ERR_SHAPE,
                  "%s: each operand must be smaller than 2 GiB (buffer offsets are 32-bit)", name);
    LFM2Q_REQUIRE((long)((M + 63) / 64) * ((N + 63) / 64) < (1L << 31), LFM2Q_ERR_SHAPE, "%s: too many tiles", name);
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

extern "C" size_t lfm2q_gemm_workspace_bytes(void) { return GEMM_WS_BYTES; }

extern "C" int lfm2q_gemm_i8_ex(const int8_t *A, const float *sa, const int8_t *B, const float *sb,
                                const lfm2q_bf16 *bias, lfm2q_bf16 *Y, int M, int N, int K, int gelu, void *ws,
                                size_t ws_bytes, lfm2q_stream_t stream) {
    if (int st = check_gemm("gemm_i8", A, B, Y, M, N, K)) return st;
    LFM2Q_REQUIRE(sa && sb, LFM2Q_ERR_ARG, "gemm_i8: sx and sw are required");
    LFM2Q_REQUIRE(!ws || (((uintptr_t)ws & 255) == 0 && ws_bytes >= 4 * (size_t)SPLIT_CNT_WORDS), LFM2Q_ERR_ARG,
                  "gemm_i8_ex: workspace must be 256-byte aligned and at least %zu bytes", 4 * (size_t)SPLIT_CNT_WORDS);
    if (gelu)
        launch_gemm<OUT_BF16_GELU>(A, B, sa, sb, bias, Y, M, N, K, (hipStream_t)stream, ws, ws_bytes);
    else
        launch_gemm<OUT_BF16>(A, B, sa, sb, bias, Y, M, N, K, (hipStream_t)stream, ws, ws_bytes);
    return launch_status("gemm_i8");
}

extern "C" int lfm2q_gemm_i8_bf16a(const lfm2q_bf16 *X, float *sa, const int8_t *B, const float *sb,
                                   const lfm2q_bf16 *bias, lfm2q_bf16 *Y, int M, int N, int K, int gelu,
                                   lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(X && sa && B && sb && Y, LFM2Q_ERR_ARG, "gemm_i8_bf16a: null pointer");
    LFM2Q_REQUIRE(M >= 1 && N >= 1 && K >= 16 && K % 16 == 0, LFM2Q_ERR_SHAPE,
                  "gemm_i8_bf16a: need M, N >= 1, K >= 16 and K %% 16 == 0 (M=%d N=%d K=%d)", M, N, K);
    LFM2Q_REQUIRE((long)M * K * 2 < (1L << 31) && (long)N * K < (1L << 31), LFM2Q_ERR_SHAPE,
                  "gemm_i8_bf16a: each operand must be smaller than 2 GiB (buffer offsets are 32-bit)");
    LFM2Q_REQUIRE(aligned16(X) && aligned16(B) && ((uintptr_t)sa & 3) == 0, LFM2Q_ERR_ALIGN,
                  "gemm_i8_bf16a: X and B must be 16-byte aligned");
    const hipStream_t st = (hipStream_t)stream;
    if (int e = launch_row_scales(X, sa, M, K, st)) return e;
    if (gelu)
        launch_gemm_bf16a<OUT_BF16_GELU>(X, B, sa, sb, bias, Y, M, N, K, st);
    else
        launch_gemm_bf16a<OUT_BF16>(X, B, sa, sb, bias, Y, M, N, K, st);
    return launch_status("gemm_i8_bf16a");
}

extern "C" int lfm2q_gemm_i8_fq(const lfm2q_bf16 *X, int8_t *q, float *sa, const int8_t *B, const float *sb,
                                const lfm2q_bf16 *bias, lfm2q_bf16 *Y, int M, int N, int K, int gelu, void *ws,
                                size_t ws_bytes, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(X && q && sa && B && sb && Y && ws, LFM2Q_ERR_ARG, "gemm_i8_fq: null pointer");
    if (int st = check_gemm("gemm_i8_fq", q, B, Y, M, N, K)) return st;
    LFM2Q_REQUIRE((long)M * K * 2 < (1L << 31), LFM2Q_ERR_SHAPE, "gemm_i8_fq: x must be smaller than 2 GiB");
    LFM2Q_REQUIRE(aligned16(X) && ((uintptr_t)sa & 3) == 0, LFM2Q_ERR_ALIGN,
                  "gemm_i8_fq: x must be 16-byte and sa 4-byte aligned");
    LFM2Q_REQUIRE(((uintptr_t)ws & 255) == 0 && ws_bytes >= GEMM_WS_BYTES, LFM2Q_ERR_ARG,
                  "gemm_i8_fq: workspace must be 256-byte aligned and at least %zu bytes", GEMM_WS_BYTES);
    const hipStream_t st = (hipStream_t)stream;
    if (!fq_applies(M, N, K, Y, bias)) {  // the pair: quant_rows, then the GEMM
        if (int e = lfm2q_quant_rows(X, q, sa, M, K, stream)) return e;
        return lfm2q_gemm_i8_ex(q, sa, B, sb, bias, Y, M, N, K, gelu, ws, ws_bytes, stream);
    }
    if (gelu)
        launch_gemm_fq<OUT_BF16_GELU>(X, q, sa, B, sb, bias, Y, M, N, K, st, ws);
    else
        launch_gemm_fq<OUT_BF16>(X, q, sa, B, sb, bias, Y, M, N, K, st, ws);
    return launch_status("gemm_i8_fq");
}

extern "C" int lfm2q_gemm_i8_grouped(const int8_t *A, const float *saT, const int8_t *B, const float *sb,
                                     const lfm2q_bf16 *bias, lfm2q_bf16 *Y, int M, int N, int K, int gelu,
                                     lfm2q_stream_t stream) {
    if (int st = check_gemm("gemm_i8", A, B, Y, M, N, K)) return st;
    LFM2Q_REQUIRE(saT && sb, LFM2Q_ERR_ARG, "gemm_i8: sxT and sw are required");
    LFM2Q_REQUIRE(K % 64 == 0, LFM2Q_ERR_SHAPE, "gemm_i8: grouped activation scales need K %% 64 == 0 (K=%d)", K);
    LFM2Q_REQUIRE((long)(K / 64) * M * 4 < (1L << 31), LFM2Q_ERR_SHAPE, "gemm_i8: sxT must be smaller than 2 GiB");
    if (gelu)
        launch_gemm_grouped<OUT_BF16_GELU>(A, B, saT, sb, bias, Y, nullptr, M, N, K, (hipStream_t)stream);
    else
        launch_gemm_grouped<OUT_BF16>(A, B, saT, sb, bias, Y, nullptr, M, N, K, (hipStream_t)stream);
    return launch_status("gemm_i8");
}

extern "C" int lfm2q_gemm_i8_q(const int8_t *A, const float *saT, const int8_t *B, const float *sb,
                               const lfm2q_bf16 *bias, int8_t *Yq, float *YsT, int M, int N, int K, int gelu,
                               lfm2q_stream_t stream) {
    if (int st = check_gemm("gemm_i8_q", A, B, Yq, M, N, K)) return st;
    LFM2Q_REQUIRE(saT && sb && YsT, LFM2Q_ERR_ARG, "gemm_i8_q: sxT, sw and ysT are required");
    LFM2Q_REQUIRE(K % 64 == 0 && N % 64 == 0, LFM2Q_ERR_SHAPE, "gemm_i8_q: need K %% 64 == 0 and N %% 64 == 0 (N=%d K=%d)",
                  N, K);
    LFM2Q_REQUIRE((long)(K / 64) * M * 4 < (1L << 31), LFM2Q_ERR_SHAPE, "gemm_i8_q: sxT must be smaller than 2 GiB");
    LFM2Q_REQUIRE(aligned16(sb) && ((uintptr_t)bias & 7) == 0 && ((uintptr_t)Yq & 7) == 0, LFM2Q_ERR_ALIGN,
                  "gemm_i8_q: sw must be 16-byte, bias and yq 8-byte aligned");
    if (gelu)
        launch_gemm_grouped<OUT_Q8_GELU>(A, B, saT, sb, bias, Yq, YsT, M, N, K, (hipStream_t)stream);
    else
        launch_gemm_grouped<OUT_Q8>(A, B, saT, sb, bias, Yq, YsT, M, N, K, (hipStream_t)stream);
    return launch_status("gemm_i8_q");
}

extern "C" int lfm2q_gemm_w8(const lfm2q_bf16 *X, const int8_t *W, const float *sw, const lfm2q_bf16 *bias,
                             lfm2q_bf16 *Y, int M, int N, int K, int gelu, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(X && W && sw && Y, LFM2Q_ERR_ARG, "gemm_w8: null pointer");
    LFM2Q_REQUIRE(M >= 1 && N >= 1 && K >= 16 && K % 16 == 0, LFM2Q_ERR_SHAPE,
                  "gemm_w8: need M, N >= 1 and K %% 16 == 0 (M=%d N=%d K=%d)", M, N, K);
    LFM2Q_REQUIRE((long)M * K * 2 < (1L << 31) && (long)N * K < (1L << 31), LFM2Q_ERR_SHAPE,
                  "gemm_w8: each operand must be smaller than 2 GiB (buffer offsets are 32-bit)");
    LFM2Q_REQUIRE(aligned16(X) && aligned16(W), LFM2Q_ERR_ALIGN, "gemm_w8: x and w must be 16-byte aligned");
    if (gelu)
        launch_gemm_w8<OUT_BF16_GELU>(X, W, sw, bias, Y, M, N, K, (hipStream_t)stream);
    else
        launch_gemm_w8<OUT_BF16>(X, W, sw, bias, Y, M, N, K, (hipStream_t)stream);
    return launch_status("gemm_w8");
}

extern "C" int lfm2q_gemm_w8_ex(const lfm2q_bf16 *X, const int8_t *W, const float *sw, const lfm2q_bf16 *bias,
                                lfm2q_bf16 *Y, int M, int N, int K, int gelu, void *ws, size_t ws_bytes,
                                lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(X && W && sw && Y, LFM2Q_ERR_ARG, "gemm_w8: null pointer");
    LFM2Q_REQUIRE(M >= 1 && N >= 1 && K >= 16 && K % 16 == 0, LFM2Q_ERR_SHAPE,
                  "gemm_w8: need M, N >= 1 and K %% 16 == 0 (M=%d N=%d K=%d)", M, N, K);
    LFM2Q_REQUIRE((long)M * K * 2 < (1L << 31) && (long)N * K < (1L << 31), LFM2Q_ERR_SHAPE,
                  "gemm_w8: each operand must be smaller than 2 GiB (buffer offsets are 32-bit)");
    LFM2Q_REQUIRE(aligned16(X) && aligned16(W), LFM2Q_ERR_ALIGN, "gemm_w8: x and w must be 16-byte aligned");
    LFM2Q_REQUIRE(!ws || (((uintptr_t)ws & 255) == 0 && ws_bytes >= 4 * (size_t)SPLIT_CNT_WORDS), LFM2Q_ERR_ARG,
                  "gemm_w8_ex: workspace must be 256-byte aligned and at least %zu bytes", 4 * (size_t)SPLIT_CNT_WORDS);
    if (gelu)
        launch_gemm_w8<OUT_BF16_GELU>(X, W, sw, bias, Y, M, N, K, (hipStream_t)stream, ws, ws_bytes);
    else
        launch_gemm_w8<OUT_BF16>(X, W, sw, bias, Y, M, N, K, (hipStream_t)stream, ws, ws_bytes);
    return launch_status("gemm_w8");
}

extern "C" int lfm2q_gemm_i8_i32(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K,
                                 lfm2q_stream_t stream) {
    if (int st = check_gemm("gemm_i8_i32", A, B, C, M, N, K)) return st;
    launch_gemm<OUT_I32>(A, B, nullptr, nullptr, nullptr, C, M, N, K, (hipStream_t)stream);
    return launch_status("gemm_i8_i32");
}

