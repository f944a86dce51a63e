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
