"""Writes the golden fixtures of tests/golden/*.npz from the pinned CPU oracle (oracle/).

Each fixture holds one small seeded case: its inputs and the oracle's outputs. They let the GPU tests check the
library without rebuilding the oracle's answers, and test_golden.py re-derives every one of them on the CPU so a
change in the oracle cannot go unnoticed. Run from the repository root:

    python tests/golden/make_golden.py
"""

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent


def bf16(a):
    return oracle.f2bf(np.asarray(a, np.float32))


def case_gemv_w8(seed, B, N, K):
    r = np.random.default_rng(seed)
    W = r.integers(-127, 128, (N, K), dtype=np.int8)
    scale = (np.abs(r.standard_normal(N)) * 0.01 + 1e-3).astype(np.float32)
    x = bf16(r.standard_normal((B, K)))
    return dict(W=W, scale=scale, x=x, y=oracle.gemv(W, scale, x))


def case_gemv_bf16(seed, B, N, K):
    r = np.random.default_rng(seed)
    W = bf16(r.standard_normal((N, K)) * 0.02)
    x = bf16(r.standard_normal((B, K)))
    return dict(W=W, x=x, y=oracle.gemv(W, None, x))


def case_swiglu_w8(seed, B, S, K):
    r = np.random.default_rng(seed)
    W = r.integers(-127, 128, (2 * S, K), dtype=np.int8)
    scale = (np.abs(r.standard_normal(2 * S)) * 0.01 + 1e-3).astype(np.float32)
    x = bf16(r.standard_normal((B, K)))
    return dict(W=W, scale=scale, x=x, y=oracle.gemv_swiglu(W, scale, x))


def case_residual_w8(seed, B, N, K):
    r = np.random.default_rng(seed)
    W = r.integers(-127, 128, (N, K), dtype=np.int8)
    scale = (np.abs(r.standard_normal(N)) * 0.01 + 1e-3).astype(np.float32)
    x = bf16(r.standard_normal((B, K)))
    h = bf16(r.standard_normal((B, N)) * 4)
    return dict(W=W, scale=scale, x=x, h=h, h_out=oracle.gemv_residual(W, scale, x, h))


def case_silu_mul(seed, B, I):
    r = np.random.default_rng(seed)
    g = bf16(r.standard_normal((B, 2 * I)) * 3)
    return dict(g=g, y=oracle.silu_mul(g))


def division_trap_rows(seed, n_rows=12):
    """Rows of 64 bf16 values holding (amax, x, -x) where x * fl(1 / s) and the correctly rounded x / s round to
    different integers (s = amax / 127): a quantizer that multiplies by the reciprocal fails them."""
    r = np.random.default_rng(seed)
    allx = np.arange(0, 0x7F80, dtype=np.uint16)
    fx = oracle.bf2f(allx)
    rows = []
    for a in np.unique(bf16(np.abs(r.standard_normal(600)) * 4 + 0.1)):
        af = oracle.bf2f(np.array([a]))[0]
        sc = np.float32(af) / np.float32(127)
        cand = fx[fx <= af]
        bad = np.nonzero(np.rint(cand / sc) != np.rint(cand * (np.float32(1) / sc)))[0]
        if bad.size:
            row = np.zeros(64, np.uint16)
            pick = allx[bad[np.linspace(0, bad.size - 1, min(bad.size, 20)).astype(int)]]
            row[0] = a
            row[1:1 + pick.size] = pick
            row[32:32 + pick.size] = pick | 0x8000
            rows.append(row)
        if len(rows) == n_rows:
            break
    return np.stack(rows)


def case_quant_rows(seed, M, K):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K)) * r.uniform(0.01, 4, (M, 1))
    x[0, 3] = 37.0
    if M > 2:
        x[2] = 0.0  # an all-zero row: s = 1e-8 / 127
    xb = bf16(x)
    if K == 64:
        xb[: min(M, 12)] = division_trap_rows(seed)[: min(M, 12)]
    q, sc = oracle.quant_rows(xb)
    return dict(x=xb, q=q, s=sc)


def case_gemm_i8(seed, M, K, N, bias, gelu):
    r = np.random.default_rng(seed)
    xq, sx = oracle.quant_rows(bf16(r.standard_normal((M, K))))
    wq, sw = oracle.quant_rows(bf16(r.standard_normal((N, K)) * 0.02))
    d = dict(xq=xq, sx=sx, wq=wq, sw=sw, acc=oracle.gemm_i8_i32(xq, wq))
    b = bf16(r.standard_normal(N)) if bias else None
    if b is not None:
        d["bias"] = b
    d["y"] = oracle.gemm_i8_epilogue(d["acc"], sx, sw, b, gelu)
    return d


def case_quant_groups(seed, M, K):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K)) * r.uniform(0.01, 4, (M, 1))
    x[0, 3] = 37.0
    if M > 2:
        x[2, :64] = 0.0  # an all-zero group: s = 1e-8 / 127
    xb = bf16(x)
    if K == 64:
        xb[: min(M, 12)] = division_trap_rows(seed)[: min(M, 12)]
    q, sT = oracle.quant_groups(xb)
    return dict(x=xb, q=q, sT=sT)


def case_add_rmsnorm(seed, rows, H, eps):
    r = np.random.default_rng(seed)
    h, y = bf16(r.standard_normal((rows, H)) * 2), bf16(r.standard_normal((rows, H)))
    w = bf16(r.random(H) + 0.5)
    hn, x = oracle.add_rmsnorm(h, y, w, eps)
    return dict(h=h, y=y, w=w, eps=np.float32(eps), h_out=hn, x=x)


def case_add_layernorm(seed, rows, D, eps):
    r = np.random.default_rng(seed)
    h, y = bf16(r.standard_normal((rows, D)) * 3), bf16(r.standard_normal((rows, D)))
    w, b = bf16(r.random(D) + 0.5), bf16(r.standard_normal(D))
    hn, x = oracle.add_layernorm(h, y, w, b, eps)
    return dict(h=h, y=y, w=w, b=b, eps=np.float32(eps), h_out=hn, x=x)


def pack_ref_int4(q):
    """q in [-8, 7] [N, K] -> uint8 [N, K/2]: weight 2j in the low nibble of byte j, stored as q + 8."""
    u = (np.asarray(q) + 8).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def pack_nibbles(v):
    """ints in [0, 15] [R, C] -> int32 [R, ceil(C/8)], nibble i of word w = column 8 w + i."""
    R, C = v.shape
    pad = np.zeros((R, -(-C // 8) * 8), np.uint32)
    pad[:, :C] = v
    w = np.zeros((R, pad.shape[1] // 8), np.uint32)
    for i in range(8):
        w |= pad[:, i::8] << np.uint32(4 * i)
    return w.view(np.int32)


def case_gemv_w4(seed, B, N, K, group):
    r = np.random.default_rng(seed)
    q = r.integers(-8, 8, (N, K))
    S = (np.abs(r.standard_normal((N, K // group))) * 0.02 + 1e-3).astype(np.float32)
    x = bf16(r.standard_normal((B, K)))
    Wp = pack_ref_int4(q)
    return dict(Wp=Wp, S=S, x=x, y=oracle.gemv_w4(Wp, S, x))


def case_gemv_w4z(seed, B, R, K, group, swiglu):
    r = np.random.default_rng(seed)
    q = r.integers(0, 16, (R, K))
    z = r.integers(0, 16, (R, K // group))
    S = (np.abs(r.standard_normal((R, K // group))) * 0.02 + 1e-3).astype(np.float16)
    x = bf16(r.standard_normal((B, K)))
    Wq, Z = pack_nibbles(q), pack_nibbles(z)
    return dict(Wq=Wq, S=S.view(np.uint16), Z=Z, x=x, y=oracle.gemv_w4z(Wq, S, Z, x, group, swiglu=swiglu))


CASES = {
    "gemv_w8_b1_n80_k1024": (case_gemv_w8, (1, 1, 80, 1024)),
    "gemv_w8_b3_n80_k1024": (case_gemv_w8, (2, 3, 80, 1024)),
    "gemv_w8_b16_n48_k2048": (case_gemv_w8, (3, 16, 48, 2048)),
    "gemv_w8_b20_n40_k512": (case_gemv_w8, (4, 20, 40, 512)),
    "gemv_bf16_b1_n48_k512": (case_gemv_bf16, (5, 1, 48, 512)),
    "gemv_bf16_b5_n48_k512": (case_gemv_bf16, (6, 5, 48, 512)),
    "swiglu_w8_b1_s40_k512": (case_swiglu_w8, (7, 1, 40, 512)),
    "swiglu_w8_b4_s48_k1024": (case_swiglu_w8, (8, 4, 48, 1024)),
    "residual_w8_b1_n64_k2048": (case_residual_w8, (9, 1, 64, 2048)),
    "residual_w8_b16_n64_k1024": (case_residual_w8, (10, 16, 64, 1024)),
    "silu_mul_b3_i300": (case_silu_mul, (11, 3, 300)),
    "quant_rows_traps_k64": (case_quant_rows, (12, 12, 64)),
    "quant_rows_m37_k1152": (case_quant_rows, (13, 37, 1152)),
    "quant_rows_m5_k4304": (case_quant_rows, (14, 5, 4304)),
    "quant_rows_m3_k8192": (case_quant_rows, (15, 3, 8192)),
    "gemm_i8_m37_k320_n24_bias": (case_gemm_i8, (16, 37, 320, 24, True, False)),
    "gemm_i8_m70_k1152_n100": (case_gemm_i8, (17, 70, 1152, 100, False, False)),
    "gemm_i8_m33_k576_n40_bias_gelu": (case_gemm_i8, (18, 33, 576, 40, True, True)),
    "gemm_i8_m129_k4304_n72_bias": (case_gemm_i8, (19, 129, 4304, 72, True, False)),
    "gemv_w4_b1_n80_k1024_g128": (case_gemv_w4, (20, 1, 80, 1024, 128)),
    "gemv_w4_b4_n48_k2048_g128": (case_gemv_w4, (21, 4, 48, 2048, 128)),
    "gemv_w4_b2_n40_k512_g64": (case_gemv_w4, (22, 2, 40, 512, 64)),
    "gemv_w4z_b1_r64_k2048_g128": (case_gemv_w4z, (23, 1, 64, 2048, 128, False)),
    "gemv_w4z_b8_r96_k1024_g128_swiglu": (case_gemv_w4z, (24, 8, 96, 1024, 128, True)),
    "quant_groups_traps_k64": (case_quant_groups, (25, 12, 64)),
    "quant_groups_m37_k1152": (case_quant_groups, (26, 37, 1152)),
    "add_rmsnorm_r9_h512": (case_add_rmsnorm, (27, 9, 512, 1e-5)),
    "add_layernorm_r7_d1152": (case_add_layernorm, (28, 7, 1152, 1e-6)),
}


def build(name):
    fn, args = CASES[name]
    return fn(*args)


def main():
    for name in CASES:
        np.savez_compressed(OUT / f"{name}.npz", **build(name))
        print("wrote", name)


if __name__ == "__main__":
    main()
