/* liblfm2q: the quantized matrix-multiply hot path of the LFM2.5-VL inference stack, as hand-written gfx950
 * (MI355X) kernels behind a C ABI.
 *
 * Conventions shared by every entry point:
 *   - All tensors are row-major and contiguous, in device memory; the caller owns every buffer. No entry point
 *     allocates, synchronizes or reads device memory on the host.
 *   - bf16 tensors are passed as their raw 16-bit patterns (lfm2q_bf16 = uint16_t).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and runs asynchronously.
 *   - The return value is a status: LFM2Q_OK (0) or one of the error codes below, in which case nothing was
 *     launched and lfm2q_last_error() returns a message for the calling thread. Argument errors are detected
 *     before any launch; LFM2Q_ERR_LAUNCH reports a failed kernel launch (hipGetLastError).
 *
 * Reference interfaces: the raw-pointer launchers of kernels/lfm2_decode.cu and kernels/int8_gemm.cu and the
 * pybind11 functions of kernels/lfm2_decode.cpp and kernels/int8_gemm.cpp (paths relative to the reference
 * repository). Each declaration cites the one it replaces.
 */
#ifndef LFM2Q_H
#define LFM2Q_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t lfm2q_bf16;
typedef void *lfm2q_stream_t; /* hipStream_t */

enum {
    LFM2Q_OK = 0,
    LFM2Q_ERR_ARG = 1,     /* null pointer, bad enum value */
    LFM2Q_ERR_SHAPE = 2,   /* sizes out of range or not multiples of what the kernel needs */
    LFM2Q_ERR_ALIGN = 3,   /* a pointer is not aligned to 16 bytes */
    LFM2Q_ERR_LAUNCH = 4,  /* the kernel launch failed */
    LFM2Q_ERR_DEVICE = 5   /* no usable device / device query failed */
};

/* Message of the last failing call on this thread ("" if none). */
const char *lfm2q_last_error(void);
/* Library version string. */
const char *lfm2q_version(void);

/* Tuning knobs: force one launch configuration of a kernel family that is otherwise chosen automatically (tile,
 * K split, kernel form, wavefronts per CU), e.g. lfm2q_set_tuning("LFM2Q_GEMM_BM", "128"). value = 1 to 4
 * comma-separated integers, or NULL / "" for automatic. A knob starts from the environment variable of the same
 * name (read once, at the first launch) and is read with one atomic load per launch. Results may differ in the last
 * bits between configurations where a kernel's summation order depends on them (the GEMV launch shapes); the W8A8
 * int32 paths are exact whatever the configuration. Knob names:
 * LFM2Q_GEMV_{WPC, PERSIST, R, VALU, MFMA, CHUNK, XS}, LFM2Q_W4_{WPC, ONESHOT, MFMA, B1_MFMA},
 * LFM2Q_GEMM_{BM, BN, KSPLIT, SWZ, BIGP, RING, STAGES, SPLITK, FQ, FQ_WAIT_US, GSEQ}, LFM2Q_CHAIN_{WAIT_MS},
 * LFM2Q_QUANT_{WG}.
 * Replaces the reference's implementation switches: set_gemv_impl() (kernels/lfm2_decode.cu:662-663, bound at
 * kernels/lfm2_decode.cpp:166) and the LFM2_INT8_BM tile override (kernels/int8_gemm.cu:691). */
int lfm2q_set_tuning(const char *name, const char *value);
/* Current value of a knob: count = number of values set (0 = automatic), values[0..3]. */
int lfm2q_get_tuning(const char *name, int *values, int *count);

/* ------------------------------------------------------------------------------------------ decode GEMVs */

/* Weight-only INT8 GEMV: y[b, n] = bf16( (sum_k W[n, k] * x[b, k]) * scale[n] ).
 * W int8 [N, K], scale fp32 [N], x bf16 [B, K], y bf16 [B, N]; B >= 1, K % 64 == 0.
 * rows: output rows per wavefront for B == 1 (1, 2 or 4; 0 = automatic), ignored otherwise.
 * Replaces launch_gemv(W, int8 = true, ...) kernels/lfm2_decode.cu:708-714 (bound as gemv(),
 * kernels/lfm2_decode.cpp:74-85). */
int lfm2q_gemv_w8(const int8_t *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *y, int B, int N, int K,
                  int rows, lfm2q_stream_t stream);

/* BF16-weight GEMV: y[b, n] = bf16( (sum_k W[n, k] * x[b, k]) * (scale ? scale[n] : 1) ).
 * W bf16 [N, K]; same shapes and rules as lfm2q_gemv_w8.
 * Replaces launch_gemv(W, int8 = false, ...) kernels/lfm2_decode.cu:708-714. */
int lfm2q_gemv_bf16(const lfm2q_bf16 *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *y, int B, int N,
                    int K, int rows, lfm2q_stream_t stream);

/* GEMV over the stacked w1|w3 weight W [2S, K] with the SwiGLU epilogue fused:
 *   g = bf16(acc[b, n] * s[n]), u = bf16(acc[b, S + n] * s[S + n]), y[b, n] = bf16( bf16(silu(g)) * u ).
 * wtype 0: W int8 (scale required); wtype 1: W bf16 (scale optional). y bf16 [B, S]; any B >= 1.
 * Bit-identical to the plain GEMV followed by lfm2q_silu_mul on the same inputs.
 * Replaces gemv_epi(0, ...) kernels/lfm2_decode.cpp:130-150 / gemv_epi_kernel<WT, 2, 0>
 * kernels/lfm2_decode.cu:724-805 (which is batch 1 only). */
int lfm2q_gemv_swiglu(int wtype, const void *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *y, int B,
                      int S, int K, lfm2q_stream_t stream);

/* GEMV with the residual add fused: h[b, n] = bf16( h[b, n] + bf16(acc[b, n] * s[n]) ), h bf16 [B, N] in place.
 * Bit-identical to the plain GEMV followed by the residual add of add_rmsnorm (kernels/lfm2_decode.cu:108-113).
 * No counterpart kernel in the reference (there it is the separate add_rmsnorm launch). */
int lfm2q_gemv_residual(int wtype, const void *W, const float *scale, const lfm2q_bf16 *x, lfm2q_bf16 *h, int B,
                        int N, int K, lfm2q_stream_t stream);

/* Batch-1 GEMV of an RMS-normalized row: x = bf16(norm_w * bf16(h * rs)), rs = 1 / sqrt(mean(h^2) + eps), computed
 * inside the GEMV, then y = x W^T s (epi 0, y bf16 [1, N]) or the SwiGLU of x over W = w1|w3 [2N, K] (epi 1,
 * y [1, N]). h and norm_w bf16 [K]; h is read, not written. Bit-identical to lfm2q_add_rmsnorm_q with no residual
 * input (its bf16 x) followed by lfm2q_gemv_w8 / lfm2q_gemv_swiglu (wtype 0: int8 W with fp32 scale, K in {1024,
 * 2048, 4096, 8192}; wtype 1: bf16 W, scale optional, K in {512, 1024, 2048, 4096}). Replaces the pair the
 * reference's decode step runs before every qkv / in_proj / w1|w3 / lm_head linear: add_rmsnorm
 * (kernels/lfm2_decode.cpp:33-38, kernel kernels/lfm2_decode.cu:96-121) then gemv / gemv_epi(0)
 * (kernels/lfm2_decode.cpp:74-85, :130-150), at the call sites src/lfm2opt/runtime.py:251-255, :276-281, :284-285. */
int lfm2q_gemv_rmsnorm(int wtype, int epi, const void *W, const float *scale, const lfm2q_bf16 *h,
                       const lfm2q_bf16 *norm_w, float eps, lfm2q_bf16 *y, int N, int K, lfm2q_stream_t stream);

/* Weight-only INT4 GEMV with group-wise scales and zero points: acc[b, n] = sum_k s[n, k/group] (q[n, k] - z[n,
 * k/group]) x[b, k] in fp32, y[b, n] = bf16(acc[b, n]) (epi 0), the SwiGLU pair of W = w1|w3 [2N, K] (epi 1, same
 * roundings as lfm2q_gemv_swiglu with the scales folded into acc) or h[b, n] = bf16(h[b, n] + bf16(acc[b, n]))
 * in place in y (epi 2). Nibble i of 32-bit word w of a weight row holds q for k = 8 w + i in both formats:
 *   fmt 0: Wq uint8 [R, K/2] holding q + 8 (weight 2j in the low nibble of byte j), S fp32 [R, K/group], Z = NULL,
 *          zero point 8 -- the reference format;
 *   fmt 1: Wq int32 [R, K/8] holding q in [0, 15], S fp16 [R, K/group], Z int32 [R, ceil(K/group/8)] with the
 *          zero point of group 8 w + j in nibble j of word w -- GPTQ-style storage;
 * R = N (2N for epi 1). x bf16 [B, K], y bf16 [B, N]; any B >= 1; group % 32 == 0, K % group == 0, K <= 8192.
 * Batches of 2..16 rows run on the matrix cores when group % 128 == 0.
 * Replaces launch_gemv_w4 kernels/lfm2_decode.cu:938-950 (bound as gemv_w4(), kernels/lfm2_decode.cpp:86-98,
 * which is fmt 0, epi 0 and batch 1 only). */
int lfm2q_gemv_w4(int fmt, const void *Wq, const void *S, const int32_t *Z, const lfm2q_bf16 *x, lfm2q_bf16 *y,
                  int B, int N, int K, int group, int epi, lfm2q_stream_t stream);

/* One GEMV of a chain: batch 1, int8 W [R, K] (R = N, or 2N = w1|w3 for epi 1) with fp32 scale [R], bf16 x [K],
 * bf16 y [N]. epi 0: y = bf16(acc * s); epi 1: the SwiGLU of lfm2q_gemv_swiglu; epi 2: y = bf16(y + bf16(acc * s))
 * in place (lfm2q_gemv_residual). */
typedef struct lfm2q_gemv_op {
    const void *W;
    const float *scale;
    const lfm2q_bf16 *x;
    lfm2q_bf16 *y;
    int32_t N, K, epi, reserved;
} lfm2q_gemv_op;

/* Bytes of the workspace lfm2q_gemv_chain needs (about 34 KiB). */
size_t lfm2q_gemv_chain_workspace_bytes(void);

/* A decode step's GEMVs as one launch: ops[0 .. n_ops-1] in order, where op j may read anything ops 0 .. j-1
 * wrote (its inputs are read only after every output of op j - 1 is written). Each output is bit-identical to the
 * separate lfm2q_gemv_w8 / lfm2q_gemv_swiglu / lfm2q_gemv_residual call on the same inputs. The weights of later
 * ops stream while an op waits for its inputs, but each op boundary still costs about 3 us of device-coherent round
 * trips: on MI355X a whole decode step as one chain is slower than the same GEMVs replayed from one HIP graph, and
 * on a par with separate eager launches.
 * ops: the table on the host (checked there); ops_dev: the same n_ops descriptors in device memory (the kernel
 * reads these; 16-byte aligned). K in {1024, 2048, 4096, 8192}, N <= 512 x the CU count, n_ops <= 128.
 * workspace: lfm2q_gemv_chain_workspace_bytes() of device memory, 256-byte aligned, zero-filled before its first
 * use and then left alone (it carries a launch counter between calls); calls sharing a workspace must be ordered
 * (one stream). Word 0 of the workspace (uint32) counts the completed launches; word 1 is set to that count (the
 * launch's own number + 1) when a dependency wait of a launch runs out (20 ms, e.g. because not every workgroup of
 * the launch could be resident; the bound is the knob LFM2Q_CHAIN_WAIT_MS): after a launch, word 1 == word 0 means
 * that launch's outputs are undefined. An expired launch does not affect the launches after it.
 * No counterpart entry point in the reference, which chains separate launches with programmatic dependent launch
 * (kernels/lfm2_decode.cu:24-62, the weight prefetch before the dependency wait at :500-512, :600-609). */
int lfm2q_gemv_chain(const lfm2q_gemv_op *ops, const lfm2q_gemv_op *ops_dev, int n_ops, void *workspace,
                     size_t workspace_bytes, lfm2q_stream_t stream);

/* lfm2q_gemv_chain without a workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc); it allocates nothing and calls no
 * allocating routine. No counterpart in the reference. Its workspace is a fixed array of
 * lfm2q_gemv_chain_workspace_bytes() (34944) bytes in the library's device memory, one per GPU, held until the
 * process ends; every call first zeroes it with a fill kernel on `stream`, so two calls on one GPU must not overlap
 * (calls on different streams at once race on the array). Limits as lfm2q_gemv_chain: 1 <= n_ops <= 128 (beyond
 * that LFM2Q_ERR_SHAPE), K in {1024, 2048, 4096, 8192}, N <= 512 x the CU count, at most 1024 CUs.
 * status: optional (NULL or a device uint32, 4-byte aligned), set at the end of the launch to 0, or nonzero if a
 * dependency wait ran out (the outputs are then undefined). Outputs are bit-identical to lfm2q_gemv_chain's. */
int lfm2q_gemv_chain_noalloc(const lfm2q_gemv_op *ops, const lfm2q_gemv_op *ops_dev, int n_ops, uint32_t *status,
                             lfm2q_stream_t stream);

/* y[b, i] = bf16( bf16(silu(g[b, i])) * g[b, I + i] ), g bf16 [B, 2I], y bf16 [B, I].
 * Replaces launch_silu_mul kernels/lfm2_decode.cu:954-969 (bound as silu_mul(), kernels/lfm2_decode.cpp:100-103). */
int lfm2q_silu_mul(const lfm2q_bf16 *g, lfm2q_bf16 *y, int B, int I, lfm2q_stream_t stream);

/* ------------------------------------------------------------------------------------------ W8A8 GEMM */

/* Per-token activation quantization: s[r] = max(max_k |x[r, k]|, 1e-8) / 127 (IEEE division),
 * q[r, k] = clamp(rint(x[r, k] / s[r]), -127, 127) with round-half-even. x bf16 [rows, K], q int8 [rows, K],
 * s fp32 [rows]; K % 8 == 0 (the reference accepts K % 128 == 0 and K <= 2048 only).
 * Replaces launch_quant_rows kernels/int8_gemm.cu:822-825 (bound as quant_rows(), kernels/int8_gemm.cpp:83-96). */
int lfm2q_quant_rows(const lfm2q_bf16 *x, int8_t *q, float *s, int rows, int K, lfm2q_stream_t stream);

/* Grouped activation quantization: one scale per row and group of 64 columns, sT[g, r] = max(max |x[r, 64 g ..
 * 64 g + 63]|, 1e-8) / 127 written transposed (sT fp32 [K/64, rows]), q as in lfm2q_quant_rows with that scale;
 * K % 64 == 0. Replaces launch_quant_groups kernels/int8_gemm.cu:435-474 (quant_rows() with a 2-D s,
 * kernels/int8_gemm.cpp:83-96, which also requires K % 128 == 0). */
int lfm2q_quant_groups(const lfm2q_bf16 *x, int8_t *q, float *sT, int rows, int K, lfm2q_stream_t stream);

/* Fused INT8 producers. Each computes a bf16 row x and quantizes it into q [rows, L] with per-row scales s [rows]
 * (grouped == 0) or per-row-and-64-column scales sT [L/64, rows] (grouped != 0), bit-identically to
 * lfm2q_quant_rows / lfm2q_quant_groups of x; x itself is also written when the x pointer is not NULL.
 * Row length L <= 8192, L % 8 == 0 (L % 64 == 0 when grouped).
 * add_rmsnorm_q (L = H): if y != NULL, h = bf16(h + y) in place; x = bf16(w * bf16(h * rs)),
 *   rs = 1 / sqrt(sum(h^2) / H + eps). Replaces launch_add_rmsnorm_q kernels/int8_gemm.cu:590-642 (binding
 *   add_rmsnorm_q(), kernels/int8_gemm.cpp:122-132). */
int lfm2q_add_rmsnorm_q(lfm2q_bf16 *h, const lfm2q_bf16 *y, const lfm2q_bf16 *w, int8_t *q, float *s,
                        lfm2q_bf16 *x, int rows, int H, float eps, int grouped, lfm2q_stream_t stream);
/* add_layernorm_q (L = D): if y != NULL, h = bf16(h + y) in place; x = bf16(((h - mean) * rstd) * w + b),
 * rstd = 1 / sqrt(sum((h - mean)^2) / D + eps). Replaces launch_add_layernorm_q kernels/int8_gemm.cu:529-585 (binding
 * add_layernorm_q(), kernels/int8_gemm.cpp:108-119, which requires D % 128 == 0 and D <= 2048). */
int lfm2q_add_layernorm_q(lfm2q_bf16 *h, const lfm2q_bf16 *y, const lfm2q_bf16 *w, const lfm2q_bf16 *b, int8_t *q,
                          float *s, lfm2q_bf16 *x, int rows, int D, float eps, int grouped, lfm2q_stream_t stream);
/* silu_mul_q (L = I): g bf16 [rows, 2I] = w1 | w3 outputs, x = bf16(bf16(silu(g1)) * g3) exactly as lfm2q_silu_mul.
 * Replaces launch_silu_mul_q kernels/int8_gemm.cu:646-682 (binding silu_mul_q(), kernels/int8_gemm.cpp:135-141). */
int lfm2q_silu_mul_q(const lfm2q_bf16 *g, int8_t *q, float *s, lfm2q_bf16 *x, int rows, int I, int grouped,
                     lfm2q_stream_t stream);

/* W8A8 GEMM with the dequant epilogue: Y[m, n] = bf16( g( ((float)acc[m, n] * sa[m]) * sb[n] + bias[n] ) ),
 * acc[m, n] = sum_k A[m, k] B[n, k] exact in int32, the three fp32 operations separately rounded (no FMA),
 * g = GELU (tanh approximation) if gelu != 0, else identity. A int8 [M, K], sa fp32 [M], B int8 [N, K],
 * sb fp32 [N], bias bf16 [N] or NULL, Y bf16 [M, N]; K % 16 == 0, any M, N >= 1.
 * Replaces launch_gemm_i8(..., grouped = false, ...) kernels/int8_gemm.cu:741-748 (bound as gemm_i8(),
 * kernels/int8_gemm.cpp:39-50, which also requires N % 8 == 0). */
int lfm2q_gemm_i8(const int8_t *A, const float *sa, const int8_t *B, const float *sb, const lfm2q_bf16 *bias,
                  lfm2q_bf16 *Y, int M, int N, int K, int gelu, lfm2q_stream_t stream);

/* lfm2q_gemm_i8 with a workspace: where the output tiles are fewer than the CUs (few tokens, narrow N) the
 * persistent 256 x 128 / 128 x 128 / 128 x 64 kernels may also cut K into 2..8 slices over workgroups; each slice's
 * int32 accumulators go to the workspace and the last workgroup of a tile adds them (exact) before the epilogue, so
 * Y is bit-identical to lfm2q_gemm_i8's. ws: lfm2q_gemm_workspace_bytes() of device memory (or at least 64 KiB: a
 * smaller one only limits the slices), 256-byte aligned, zero-filled before its first use; every call that returns
 * 0 leaves its counters zero again. Calls sharing a workspace must not overlap (one stream, or ordered); ws NULL is
 * lfm2q_gemm_i8. No counterpart in the reference (added for the K split). */
int lfm2q_gemm_i8_ex(const int8_t *A, const float *sa, const int8_t *B, const float *sb, const lfm2q_bf16 *bias,
                     lfm2q_bf16 *Y, int M, int N, int K, int gelu, void *ws, size_t ws_bytes, lfm2q_stream_t stream);

/* Bytes of the lfm2q_gemm_i8_ex / lfm2q_gemm_w8_ex / lfm2q_gemm_i8_fq workspace (64 MiB + 320 KiB). */
size_t lfm2q_gemm_workspace_bytes(void);

/* The per-token W8A8 layer on bf16 activations: q int8 [M, K] and sa fp32 [M] receive X's per-token quantization
 * (the bytes lfm2q_quant_rows writes) and Y the GEMM on them; Y, q and sa equal lfm2q_quant_rows followed by
 * lfm2q_gemm_i8_ex bit for bit. By default the call runs exactly that pair (the faster form on MI355X). With the
 * tuning knob LFM2Q_GEMM_FQ = 1 it runs them as one launch where the shape fits the persistent GEMM (K <= 16384,
 * N % 8 == 0, Y 16-byte aligned, M K and M N below 2^30): the workgroups first quantize X together, in chunks of
 * rows, each waiting until every chunk is written (a workgroup that waits longer than LFM2Q_GEMM_FQ_WAIT_US, 20 us
 * by default, quantizes the open chunks itself), then run the GEMM's tiles. ws: the lfm2q_gemm_i8_ex workspace at
 * its full size (lfm2q_gemm_workspace_bytes()), 256-byte aligned, zero-filled before its first use; its last
 * 256 KiB hold the one-launch form's control block, which every call leaves valid. Calls sharing a workspace must
 * not overlap. Shapes, alignment, B, sb, bias, gelu as in lfm2q_gemm_i8; X and q 16-byte aligned.
 * The reference runs the pair as two kernels (quantize_rows then gemm_i8: src/lfm2opt/int8.py:45-51,
 * kernels/int8_gemm.cu:391-432 then :125-297); this entry point is the pair behind one call. */
int lfm2q_gemm_i8_fq(const lfm2q_bf16 *X, int8_t *q, float *sa, const int8_t *B, const float *sb,
                     const lfm2q_bf16 *bias, lfm2q_bf16 *Y, int M, int N, int K, int gelu, void *ws, size_t ws_bytes,
                     lfm2q_stream_t stream);

/* W8A8 GEMM on bf16 activations, quantized per token inside the GEMM: a first pass writes sa fp32 [M], the
 * scales lfm2q_quant_rows would write for X, and the GEMM quantizes each stage of X bf16 [M, K] on its way into
 * LDS with the quantizers' own code, so Y equals lfm2q_quant_rows + lfm2q_gemm_i8 on the same inputs bit for bit,
 * without the int8 copy of X. K % 16 == 0; B, sb, bias, Y, gelu as in lfm2q_gemm_i8. Tiles of at most 128 x 128.
 * The reference's per-token path runs quantize_rows and gemm_i8 as two kernels (src/lfm2opt/int8.py:45-51,
 * kernels/int8_gemm.cu:391-432 then :125-297); this is the fused form of that pair. */
int lfm2q_gemm_i8_bf16a(const lfm2q_bf16 *X, float *sa, const int8_t *B, const float *sb, const lfm2q_bf16 *bias,
                        lfm2q_bf16 *Y, int M, int N, int K, int gelu, lfm2q_stream_t stream);

/* W8A8 GEMM with grouped-64 activation scales saT fp32 [K/64, M] (lfm2q_quant_groups' layout): per 64-wide K group g
 * the exact int32 partial sum folds into fp32 as facc = fma((float)part_g, saT[g, m], facc) in group order, then
 * Y[m, n] = bf16( gelu?( facc * sb[n] + bias[n] ) ) (two separately rounded ops). K % 64 == 0.
 * Replaces launch_gemm_i8(..., grouped = true, ...) kernels/int8_gemm.cu:741-748 (gemm_i8() with a 2-D sx). */
int lfm2q_gemm_i8_grouped(const int8_t *A, const float *saT, const int8_t *B, const float *sb, const lfm2q_bf16 *bias,
                          lfm2q_bf16 *Y, int M, int N, int K, int gelu, lfm2q_stream_t stream);

/* The grouped W8A8 GEMM writing the next W8A8 GEMM's input: the bf16 values lfm2q_gemm_i8_grouped would write are
 * quantized per row and group of 64 columns exactly as lfm2q_quant_groups does, into Yq int8 [M, N] and
 * YsT fp32 [N/64, M]. K % 64 == 0, N % 64 == 0; sb 16-byte, bias and Yq 8-byte aligned.
 * Replaces launch_gemm_i8_q kernels/int8_gemm.cu:750-760 (binding gemm_i8_q(), kernels/int8_gemm.cpp:53-69, which
 * requires N % 128 == 0). */
int lfm2q_gemm_i8_q(const int8_t *A, const float *saT, const int8_t *B, const float *sb, const lfm2q_bf16 *bias,
                    int8_t *Yq, float *YsT, int M, int N, int K, int gelu, lfm2q_stream_t stream);

/* W8A16 GEMM: Y[m, n] = bf16( g( acc[m, n] * sw[n] + bias[n] ) ), acc = sum_k X[m, k] W[n, k] accumulated in fp32
 * on the bf16 matrix cores (int8 weights converted exactly), g = GELU-tanh if gelu != 0. X bf16 [M, K], W int8 [N, K],
 * sw fp32 [N], bias bf16 [N] or NULL, Y bf16 [M, N]; K % 16 == 0. Replaces launch_gemm_w8
 * kernels/int8_gemm.cu:762-771 (binding gemm_w8(), kernels/int8_gemm.cpp:72-79). */
int lfm2q_gemm_w8(const lfm2q_bf16 *X, const int8_t *W, const float *sw, const lfm2q_bf16 *bias, lfm2q_bf16 *Y, int M,
                  int N, int K, int gelu, lfm2q_stream_t stream);

/* lfm2q_gemm_w8 with a workspace (the lfm2q_gemm_i8_ex one: lfm2q_gemm_workspace_bytes(), zero-filled before its
 * first use, left with its counters zero by every call that returns 0, not shared by overlapping calls): where the
 * tiles leave more than half the CUs idle, K is also cut into up to 8 slices over workgroups and the last workgroup
 * of each tile sums the slices' fp32 tiles in slice order (so the result does not depend on which came last; its
 * last bits differ from lfm2q_gemm_w8's, within the same tolerance). ws NULL is lfm2q_gemm_w8. No counterpart in the
 * reference (added for the K split). */
int lfm2q_gemm_w8_ex(const lfm2q_bf16 *X, const int8_t *W, const float *sw, const lfm2q_bf16 *bias, lfm2q_bf16 *Y,
                     int M, int N, int K, int gelu, void *ws, size_t ws_bytes, lfm2q_stream_t stream);

/* The exact int32 accumulators of the W8A8 GEMM: C[m, n] = sum_k A[m, k] B[n, k], C int32 [M, N]. No counterpart
 * entry point in the reference (whose tests use torch._int_mm for this, tests/test_int8_gemm.py:236). */
int lfm2q_gemm_i8_i32(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, lfm2q_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LFM2Q_H */
