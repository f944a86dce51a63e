/* CPU oracle for the quantized matrix-multiply hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, in plain C, the arithmetic of the reference repository's kernels
 * and test references so that the GPU library can be checked against it. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the reference results are compared with (or, in the
 * baseline, as the timed CPU path); the product (liblfm2q + lfm2opt) never calls it.
 *
 * Built with -ffp-contract=off and without fast-math: every fp32 operation below rounds exactly once, in the
 * order written, like the reference's __fmul_rn / __fadd_rn sequences. bf16 values are raw uint16 patterns.
 * Reference paths are relative to the reference repository root.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ bf16 */
static inline float bf2f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* round to nearest even (torch's .to(torch.bfloat16), CUDA __float2bfloat16_rn); NaN -> quiet NaN */
static inline uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static inline float rbf(float f) { return bf2f(f2bf(f)); }

uint16_t orc_f2bf(float f) { return f2bf(f); }
float orc_bf2f(uint16_t h) { return bf2f(h); }

void orc_f2bf_array(const float *x, int64_t n, uint16_t *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = f2bf(x[i]);
}

/* ------------------------------------------------------------------------------------------ elementwise */
/* silu as the decode kernels compute it: g / (1 + exp(-g)) in fp32 (kernels/lfm2_decode.cu:962) */
static inline float silu(float g) { return g / (1.0f + expf(-g)); }
/* GELU tanh approximation in fp32 (kernels/int8_gemm.cu:87-89, = F.gelu(approximate="tanh")) */
static inline float gelu_tanh(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

float orc_silu(float g) { return silu(g); }
float orc_gelu_tanh(float v) { return gelu_tanh(v); }

/* y[b, i] = bf16(bf16(silu(a)) * u) on g = [B, 2I] = a | u (kernels/lfm2_decode.cu:954-963) */
void orc_silu_mul(const uint16_t *g, int64_t B, int64_t I, uint16_t *y) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t i = 0; i < I; ++i) {
            const float a = bf2f(g[b * 2 * I + i]), u = bf2f(g[b * 2 * I + I + i]);
            y[b * I + i] = f2bf(rbf(silu(a)) * u);
        }
}

/* ------------------------------------------------------------------------------------------ activation quant */
/* one symmetric scale per row: s = max(amax, 1e-8) / 127 (true division), q = clamp(rint(x / s), -127, 127),
 * rint = round half to even (tests/test_int8_gemm.py:35-38 ref_quant; kernels/int8_gemm.cu:391-432) */
static inline int8_t q8(float v, float sc) {
    float r = rintf(v / sc);
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    return (int8_t)r;
}

void orc_quant_rows(const uint16_t *x, int64_t rows, int64_t K, int8_t *q, float *s) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * K;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) amax = fmaxf(amax, fabsf(bf2f(xr[k])));
        const float sc = fmaxf(amax, 1e-8f) / 127.0f;
        s[r] = sc;
        for (int64_t k = 0; k < K; ++k) q[r * K + k] = q8(bf2f(xr[k]), sc);
    }
}

/* one scale per row and group of 64 columns, written transposed sT[K/64][rows]
 * (tests/test_int8_gemm.py:64-69 ref_quant_groups; kernels/int8_gemm.cu:435-474) */
void orc_quant_groups(const uint16_t *x, int64_t rows, int64_t K, int8_t *q, float *sT) {
    const int64_t G = K / 64;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g < G; ++g) {
            const uint16_t *xg = x + r * K + g * 64;
            float amax = 0.0f;
            for (int k = 0; k < 64; ++k) amax = fmaxf(amax, fabsf(bf2f(xg[k])));
            const float sc = fmaxf(amax, 1e-8f) / 127.0f;
            sT[g * rows + r] = sc;
            for (int k = 0; k < 64; ++k) q[r * K + g * 64 + k] = q8(bf2f(xg[k]), sc);
        }
}

/* ------------------------------------------------------------------------------------------ INT8 producers */
/* The bf16 outputs the fused INT8 producers quantize (kernels/int8_gemm.cu:527-682): the row statistics are summed
 * in fp64 and rounded to fp32 once (the kernels' fp32 reduction order is their own), everything after follows the
 * kernels' fp32 / bf16 rounding points. y (the residual input) may be NULL; h is updated in place when it is not. */

/* LM prefill, = add_rmsnorm (kernels/lfm2_decode.cu:96-121): h = bf16(h + y); ms = sum h^2 / H;
 * rs = 1 / sqrt(ms + eps) (correctly rounded); x = bf16(w * bf16(h * rs)) */
void orc_add_rmsnorm(uint16_t *h, const uint16_t *y, const uint16_t *w, int64_t rows, int64_t H, float eps,
                     uint16_t *x) {
    for (int64_t r = 0; r < rows; ++r) {
        uint16_t *hr = h + r * H;
        double ss = 0.0;
        for (int64_t i = 0; i < H; ++i) {
            if (y) hr[i] = f2bf(bf2f(hr[i]) + bf2f(y[r * H + i]));
            const double v = bf2f(hr[i]);
            ss += v * v;
        }
        const float ms = (float)ss / (float)H;
        const float rs = (float)(1.0 / sqrt((double)(ms + eps)));
        for (int64_t i = 0; i < H; ++i) x[r * H + i] = f2bf(bf2f(w[i]) * rbf(bf2f(hr[i]) * rs));
    }
}

/* vision, = add_layernorm (kernels/vision_ops.cu:29-80): h = bf16(h + y); mean = sum h / D;
 * var = sum (h - mean)^2 / D; rstd = 1 / sqrt(var + eps); x = bf16(((h - mean) * rstd) * w + b) */
void orc_add_layernorm(uint16_t *h, const uint16_t *y, const uint16_t *w, const uint16_t *b, int64_t rows,
                       int64_t D, float eps, uint16_t *x) {
    for (int64_t r = 0; r < rows; ++r) {
        uint16_t *hr = h + r * D;
        double sum = 0.0;
        for (int64_t i = 0; i < D; ++i) {
            if (y) hr[i] = f2bf(bf2f(hr[i]) + bf2f(y[r * D + i]));
            sum += bf2f(hr[i]);
        }
        const float mean = (float)sum / (float)D;
        double qs = 0.0;
        for (int64_t i = 0; i < D; ++i) {
            const double d = (double)(bf2f(hr[i]) - mean);
            qs += d * d;
        }
        const float var = (float)qs / (float)D;
        const float rstd = (float)(1.0 / sqrt((double)(var + eps)));
        for (int64_t i = 0; i < D; ++i) {
            float v = (bf2f(hr[i]) - mean) * rstd;
            v = v * bf2f(w[i]);
            x[r * D + i] = f2bf(v + bf2f(b[i]));
        }
    }
}

/* ------------------------------------------------------------------------------------------ W8A8 GEMM */
/* exact integer product C[m, n] = sum_k A[m, k] B[n, k] (A [M, K], B [N, K], both int8). |C| <= 127^2 K fits
 * int32 for K < 133144, so the int64 sum is cast without loss. */
void orc_gemm_i8_i32(const int8_t *A, const int8_t *B, int64_t M, int64_t N, int64_t K, int32_t *C) {
    for (int64_t m = 0; m < M; ++m) {
        const int8_t *a = A + m * K;
        for (int64_t n = 0; n < N; ++n) {
            const int8_t *b = B + n * K;
            int64_t acc = 0;
            for (int64_t k = 0; k < K; ++k) acc += (int32_t)a[k] * (int32_t)b[k];
            C[m * N + n] = (int32_t)acc;
        }
    }
}

/* per-token W8A8 epilogue on the exact accumulators (kernels/int8_gemm.cu:93-115 store_tile):
 *   v = ((float)acc * sx[m]) * sw[n] + b[n]   (three separately rounded fp32 ops, no FMA)
 *   y = bf16(gelu ? gelu_tanh(v) : v)
 * (float)acc rounds to nearest even, as torch's .float() of the exact fp64 sum in tests/test_int8_gemm.py:166. */
void orc_gemm_i8_epilogue(const int32_t *C, const float *sx, const float *sw, const uint16_t *bias, int64_t M,
                          int64_t N, int gelu, uint16_t *Y) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float v = (float)C[m * N + n] * sx[m];
            v = v * sw[n];
            v = v + (bias ? bf2f(bias[n]) : 0.0f);
            if (gelu) v = gelu_tanh(v);
            Y[m * N + n] = f2bf(v);
        }
}

/* grouped-64 W8A8 (kernels/int8_gemm.cu:202-230): per 64-wide K group g the exact int32 partial sum is folded
 * into fp32 with one FMA, facc = fma((float)part, sxT[g][m], facc), then v = facc * sw[n] + b[n]. */
void orc_gemm_i8_grouped(const int8_t *A, const float *sxT, const int8_t *B, const float *sw, const uint16_t *bias,
                         int64_t M, int64_t N, int64_t K, int gelu, uint16_t *Y) {
    const int64_t G = K / 64;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float facc = 0.0f;
            for (int64_t g = 0; g < G; ++g) {
                int32_t part = 0;
                for (int k = 0; k < 64; ++k) part += (int32_t)A[m * K + g * 64 + k] * (int32_t)B[n * K + g * 64 + k];
                facc = fmaf((float)part, sxT[g * M + m], facc);
            }
            float v = facc * sw[n];
            v = v + (bias ? bf2f(bias[n]) : 0.0f);
            if (gelu) v = gelu_tanh(v);
            Y[m * N + n] = f2bf(v);
        }
}

/* W8A16 (kernels/int8_gemm.cu:306-388 then store_tile with no activation scale): acc = sum_k x[m, k] w[n, k] in fp64
 * (exact products, the kernel accumulates in fp32 in its own order), rounded once to fp32, then
 * y = bf16(gelu?(acc * sw[n] + b[n])) with separately rounded ops. */
void orc_gemm_w8(const uint16_t *X, const int8_t *W, const float *sw, const uint16_t *bias, int64_t M, int64_t N,
                 int64_t K, int gelu, uint16_t *Y) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += (double)bf2f(X[m * K + k]) * (double)W[n * K + k];
            float v = (float)acc * sw[n];
            v = v + (bias ? bf2f(bias[n]) : 0.0f);
            if (gelu) v = gelu_tanh(v);
            Y[m * N + n] = f2bf(v);
        }
}

/* ------------------------------------------------------------------------------------------ decode GEMVs */
/* The GEMV accumulators are computed in fp64 (the sum of exact products) and rounded once to fp32, which is where
 * the reference kernel holds its fp32 warp sum; everything after that point follows the kernel's fp32 rounding
 * points exactly (kernels/lfm2_decode.cu:657-659, :779 and :789, :108-113). wtype 0: W int8, 1: W bf16. */
static inline double wval(const void *W, int wtype, int64_t idx) {
    return wtype == 0 ? (double)((const int8_t *)W)[idx] : (double)bf2f(((const uint16_t *)W)[idx]);
}

static float gemv_acc(const void *W, int wtype, const uint16_t *x, int64_t row, int64_t K) {
    double acc = 0.0;
    for (int64_t k = 0; k < K; ++k) acc += wval(W, wtype, row * K + k) * (double)bf2f(x[k]);
    return (float)acc;
}

static inline float scaled(float a, const float *scale, int64_t n) { return scale ? a * scale[n] : a; }

/* y[b, n] = bf16(acc * scale[n]) (gemv_direct_kernel, kernels/lfm2_decode.cu:576-661) */
void orc_gemv(const void *W, int wtype, const float *scale, const uint16_t *x, int64_t B, int64_t N, int64_t K,
              uint16_t *y) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t n = 0; n < N; ++n) y[b * N + n] = f2bf(scaled(gemv_acc(W, wtype, x + b * K, n, K), scale, n));
}

/* W = w1|w3 [2S, K]: g = bf16(acc_g s), u = bf16(acc_u s), y = bf16(bf16(silu(g)) u)
 * (gemv_epi_kernel<WT, 2, 0>, kernels/lfm2_decode.cu:779, :786-790) */
void orc_gemv_swiglu(const void *W, int wtype, const float *scale, const uint16_t *x, int64_t B, int64_t S,
                     int64_t K, uint16_t *y) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t n = 0; n < S; ++n) {
            const float g = rbf(scaled(gemv_acc(W, wtype, x + b * K, n, K), scale, n));
            const float u = rbf(scaled(gemv_acc(W, wtype, x + b * K, S + n, K), scale, S + n));
            y[b * S + n] = f2bf(rbf(silu(g)) * u);
        }
}

/* h[b, n] = bf16(h + bf16(acc s)) in place: the GEMV's bf16 output added to the residual stream exactly as
 * add_rmsnorm_kernel<true> does (kernels/lfm2_decode.cu:108-113) */
void orc_gemv_residual(const void *W, int wtype, const float *scale, const uint16_t *x, int64_t B, int64_t N,
                       int64_t K, uint16_t *h) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t n = 0; n < N; ++n) {
            const float yv = rbf(scaled(gemv_acc(W, wtype, x + b * K, n, K), scale, n));
            h[b * N + n] = f2bf(bf2f(h[b * N + n]) + yv);
        }
}

/* ------------------------------------------------------------------------------------------ INT4 GEMVs */
/* Reference format (src/lfm2opt/quant.py:21-47, kernels/lfm2_decode.cu:833-924): Wp uint8 [N, K/2], element 2j in
 * the low nibble and 2j+1 in the high nibble of byte j, stored as q + 8; S fp32 [N, K/group];
 * w = (nibble - 8) * S[n, k / group]; y = bf16(sum_k w x). */
void orc_gemv_w4(const uint8_t *Wp, const float *S, const uint16_t *x, int64_t B, int64_t N, int64_t K,
                 int64_t group, uint16_t *y) {
    const int64_t G = K / group;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const uint8_t byte = Wp[n * (K / 2) + k / 2];
                const int q = (k & 1) ? (byte >> 4) : (byte & 15);
                acc += (double)(q - 8) * (double)S[n * G + k / group] * (double)bf2f(x[b * K + k]);
            }
            y[b * N + n] = f2bf((float)acc);
        }
}

static inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-8f;
            memcpy(&u, &f, 4);
            u |= sign;
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

/* GPTQ-style asymmetric format: Wq int32 [N, K/8] (nibble i of word w holds k = 8w + i, value q in [0, 15]),
 * S fp16 [N, K/group], Z int32 [N, ceil(G/8)] (nibble j of word w = zero point of group 8w + j);
 * w = S[n, g] * (q - Z[n, g]). With Z = 8 and S exactly representable in fp16 this is the reference format.
 * epi 0: y[b, n] = bf16(acc); epi 1 (SwiGLU, W = w1|w3 [2S, K], y [B, S]): g = bf16(acc_g), u = bf16(acc_u),
 * y = bf16(bf16(silu(g)) u). */
static float w4z_acc(const int32_t *Wq, const uint16_t *S, const int32_t *Z, const uint16_t *x, int64_t row,
                     int64_t K, int64_t group) {
    const int64_t G = K / group, ZW = (G + 7) / 8;
    double acc = 0.0;
    for (int64_t k = 0; k < K; ++k) {
        const uint32_t word = (uint32_t)Wq[row * (K / 8) + k / 8];
        const int q = (word >> (4 * (k & 7))) & 15;
        const int64_t g = k / group;
        const int z = ((uint32_t)Z[row * ZW + g / 8] >> (4 * (g & 7))) & 15;
        acc += (double)f16_to_f32(S[row * G + g]) * (double)(q - z) * (double)bf2f(x[k]);
    }
    return (float)acc;
}

void orc_gemv_w4z(const int32_t *Wq, const uint16_t *S, const int32_t *Z, const uint16_t *x, int64_t B, int64_t N,
                  int64_t K, int64_t group, int epi, uint16_t *y) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t n = 0; n < N; ++n) {
            if (epi == 0) {
                y[b * N + n] = f2bf(w4z_acc(Wq, S, Z, x + b * K, n, K, group));
            } else {
                const float g = rbf(w4z_acc(Wq, S, Z, x + b * K, n, K, group));
                const float u = rbf(w4z_acc(Wq, S, Z, x + b * K, N + n, K, group));
                y[b * N + n] = f2bf(rbf(silu(g)) * u);
            }
        }
}
