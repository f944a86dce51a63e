"""Constructed W8A8 operands whose bf16 outputs depend on each fp32 rounding point of the epilogue and the grouped
fold, with the expected bits derived by hand (in the docstrings), so the oracle and the kernels are pinned to the
operation sequence itself and not only to a tolerance.

Grouped fold (kernels/int8_gemm.cu:202-215, then store_tile :93-115 with no activation scale): for each 64-wide K
group g in order, facc = fma(float(part_g), sxT[g, m], facc) with one rounding; then y = bf16(fl(fl(facc * sw[n]) +
b[n])). Per token (store_tile): y = bf16(fl(fl(fl(acc * sx[m]) * sw[n]) + b[n])), no contraction.

Every sum here is a single nonzero product (wq holds a 1 at the first column of each group), so part_g = xq[m, 64 g].
"""

import numpy as np

E23 = 2.0 ** -23
E24 = 2.0 ** -24


def f32(v):
    out = np.float32(v)
    assert float(out) == v, f"{v} is not an fp32 value"
    return out


def grouped_fold_case():
    """M = 4, K = 192 (3 groups), N = 8. Expected cells:

    - row 0, column 0 (sw = 1, b = 0): groups (-1, P) then (3, 1 + 2^-23) with P = 3 + 2^-21 = fl(3 (1 + 2^-23)) (the
      exact product 3 + 1.5 2^-22 is a tie, rounded to the even 3 + 2^-21). In order with fma: -P, then
      3 + 3 2^-23 - P = -2^-23 exactly, so y = bf16(-2^-23) = 0xb400. A fold that rounds the product first gives
      P - P = 0, and one that runs the groups backwards gives fma(-1, P, fl(3 (1 + 2^-23))) = 0.
    - row 1, column 0: groups (1, 1), (1, 2^-24), (-1, 1). In fp32, 1 + 2^-24 is a tie rounded to 1, so the fold
      ends at 1 - 1 = +0: y = 0x0000. An accumulator wider than fp32 keeps 2^-24 (0x3380).
    - row 2, column 1 (sw = 1 - 2^-24, b = -1): facc = 1 + 2^-23; the exact product 1 + 2^-24 - 2^-47 is below
      the half-way point, so fl(facc sw) = 1 and y = bf16(1 - 1) = 0x0000. An fma epilogue keeps
      2^-24 - 2^-47 and gives bf16 2^-24 = 0x3380.
    - row 2, column 0: bf16(1 + 2^-23) = 1.0 = 0x3f80.
    """
    M, K, N = 4, 192, 8
    xq = np.zeros((M, K), np.int8)
    wq = np.zeros((N, K), np.int8)
    wq[:, 0::64] = 1
    sxT = np.ones((K // 64, M), np.float32)
    xq[0, [0, 64]] = (-1, 3)
    sxT[0, 0], sxT[1, 0] = f32(3 + 2.0 ** -21), f32(1 + E23)
    xq[1, [0, 64, 128]] = (1, 1, -1)
    sxT[1, 1] = f32(E24)
    xq[2, 0] = 1
    sxT[0, 2] = f32(1 + E23)
    sw = np.ones(N, np.float32)
    sw[1] = f32(1 - E24)
    bias = np.zeros(N, np.uint16)
    bias[1] = 0xBF80  # bf16 -1.0
    expect = {(0, 0): 0xB400, (1, 0): 0x0000, (2, 1): 0x0000, (2, 0): 0x3F80}
    return xq, sxT, wq, sw, bias, expect


def per_token_epilogue_case():
    """M = 3, K = 64, N = 8, per-token scales. Expected cells:

    - row 0, column 0 (acc = 3, sx = sw = 1 + 2^-23, b = bf16(-3)): fl(3 sx) = 3 + 2^-21 (a tie, to even), then
      (3 + 2^-21)(1 + 2^-23) = 3 + 3.5 2^-22 + 2^-44 rounds up to 3 + 2^-20, and y = bf16(2^-20) = 0x3580.
      acc * fl(sx sw) instead gives 3 (1 + 2^-22) = 3 + 3 2^-22 and y = bf16(3 2^-22) = 0x3540.
    - row 1, column 1 (acc = 1, sx = 1 + 2^-23, sw = 1 - 2^-24, b = -1): fl(sx sw) = fl(1 + 2^-24 - 2^-47) = 1, so
      y = 0x0000; an fma of the last two operations gives bf16(2^-24 - 2^-47) = 0x3380.
    - row 2, column 2 (acc = -5, sx = 0.5, sw = 0.25, b = 1): -0.625 + 1 = 0.375 = 0x3ec0 (a bias added before the
      scales would give bf16(-4 x 0.125) = -0.5).
    """
    M, K, N = 3, 64, 8
    xq = np.zeros((M, K), np.int8)
    wq = np.zeros((N, K), np.int8)
    wq[:, 0] = 1
    xq[:, 0] = (3, 1, -5)
    sx = np.array([f32(1 + E23), f32(1 + E23), 0.5], np.float32)
    sw = np.ones(N, np.float32)
    sw[:3] = (f32(1 + E23), f32(1 - E24), 0.25)
    bias = np.zeros(N, np.uint16)
    bias[:3] = (0xC040, 0xBF80, 0x3F80)  # bf16 -3, -1, 1
    expect = {(0, 0): 0x3580, (1, 1): 0x0000, (2, 2): 0x3EC0}
    return xq, sx, wq, sw, bias, expect
