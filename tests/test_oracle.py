"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

The reference ships no golden vectors for this path (its tests draw fresh CUDA random tensors), so every oracle
function is pinned here by what the mathematics fixes -- closed forms on constructed inputs, known-answer bit
patterns, invariants and brute force -- and, where the reference's own test states the expected value as a torch
expression, by that expression evaluated with torch on the CPU (an implementation independent of oracle.c).
Each check is chosen so that a plausible slip (a transposed operand, a multiply by 1/s instead of a division, the
bias added before the scales, the wrong nibble order, a dropped rounding point) fails it.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
import rounding_cases

RNG = np.random.default_rng(1234)


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def from_bits(h):
    return torch.from_numpy(np.ascontiguousarray(h, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def rand_bf16(shape, scale=1.0):
    return bf16_bits(torch.from_numpy((RNG.standard_normal(shape) * scale).astype(np.float32)))


def ulps(a, b):
    """max distance in bf16 ulps between two bf16 bit arrays (sign-magnitude -> ordered integers)."""
    ia = a.astype(np.int32)
    ib = b.astype(np.int32)
    ia = np.where(ia >= 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib >= 0x8000, 0x8000 - ib, ib)
    return int(np.abs(ia - ib).max()) if ia.size else 0


def assert_gelu_close(y, v):
    """y (bf16 bits) = the reference's tanh GELU of v (fp32 tensor): within 1 bf16 ulp of torch's F.gelu, or, where
    1 + tanh(.) cancels in fp32 for v << 0 (the reference's formula; torch may return -0 there), within one fp32 ulp
    of v in absolute value, as in test_silu_gelu_against_math."""
    ref = bf16_bits(F.gelu(v, approximate="tanh"))
    ia, ib = y.astype(np.int32), ref.astype(np.int32)
    ia = np.where(ia >= 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib >= 0x8000, 0x8000 - ib, ib)
    close = np.abs(ia - ib) <= 1
    vv = v.double().numpy()
    tail = np.abs(oracle.bf2f(y).astype(np.float64) - oracle.bf2f(ref).astype(np.float64)) <= 2.0 ** -23 * np.abs(vv)
    assert np.all(close | (tail & (vv < 0))), f"{int((~(close | tail)).sum())} outputs off"


# ------------------------------------------------------------------------------------------------ bf16
def test_f2bf_known_answers():
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F808000: 0x3F80,  # 1 + 2^-8: tie -> even (down)
        0x3F818000: 0x3F82,  # 1 + 3*2^-8: tie -> even (up)
        0x3F808001: 0x3F81,  # just above the tie
        0x3F807FFF: 0x3F80,  # just below the tie
        0x80000000: 0x8000,  # -0
        0x7F800000: 0x7F80,  # inf
        0xFF800000: 0xFF80,  # -inf
        0x7F7FFFFF: 0x7F80,  # FLT_MAX rounds to inf
        0x00000001: 0x0000,  # smallest subnormal rounds to 0
    }
    for fbits, hb in cases.items():
        f = np.array([fbits], np.uint32).view(np.float32)
        assert oracle.f2bf(f)[0] == hb, hex(fbits)
    nan = oracle.f2bf(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_f2bf_matches_torch():
    x = np.concatenate([(RNG.standard_normal(200000) * 10 ** RNG.uniform(-30, 30, 200000)).astype(np.float32),
                        np.array(RNG.integers(0, 2 ** 32, 100000, dtype=np.uint64), np.uint32).view(np.float32)])
    x = x[np.isfinite(x)].astype(np.float32)
    assert np.array_equal(oracle.f2bf(x), bf16_bits(torch.from_numpy(x)))
    h = np.arange(65536, dtype=np.uint16)
    f = oracle.bf2f(h)
    ok = np.isfinite(f)
    assert np.array_equal(oracle.f2bf(f[ok]), h[ok])  # exact round trip of every finite bf16


def test_f16_decode_matches_numpy():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32_scalar(v) for v in h], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin], ref[fin]) and np.array_equal(np.isnan(got), np.isnan(ref))


def test_silu_gelu_against_math():
    for v in np.concatenate([np.linspace(-20, 20, 801), [0.0, 1e-30, -1e-30, 88.0, -88.0]]):
        v32 = float(np.float32(v))
        s = v32 / (1 + math.exp(-v32))
        assert abs(oracle.silu_scalar(v32) - s) <= 4e-7 * max(abs(s), 1e-30) + 1e-38
        g = 0.5 * v32 * (1 + math.tanh(math.sqrt(2 / math.pi) * (v32 + 0.044715 * v32 ** 3)))
        # 1 + tanh(.) cancels in fp32 for v << 0 (as in the reference's formula): absolute slack of one fp32 ulp of v
        assert abs(oracle.gelu_scalar(v32) - g) <= 2e-6 * abs(g) + 2.0 ** -23 * abs(v32)
    assert oracle.silu_scalar(0.0) == 0.0 and oracle.gelu_scalar(0.0) == 0.0


# ------------------------------------------------------------------------------------------------ quant
def test_quant_rows_power_of_two_scales_closed_form():
    """amax = 127 * 2^j makes s = 2^j exactly, so q = rint(x / 2^j) with ties to even, computable by hand."""
    for j in (-6, 0, 3):
        vals = np.array([127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, 126.5, -126.5, 0.25, 0, -127], np.float64)
        expect = np.array([127, 2, 4, -2, 0, 0, 2, 126, -126, 0, 0, -127], np.int8)
        x = bf16_bits(torch.from_numpy((vals * 2.0 ** j).astype(np.float32)))
        q, s = oracle.quant_rows(x[None, :])
        assert s[0] == np.float32(2.0 ** j)
        assert np.array_equal(q[0], expect), (j, q[0])


def test_quant_rows_zero_row_and_clamp():
    x = np.zeros((2, 128), np.uint16)
    x[1, 5] = bf16_bits(torch.tensor([1e-12]))[0]  # below the 1e-8 floor: s stays at the floor
    q, s = oracle.quant_rows(x)
    floor = np.float32(np.float32(1e-8) / np.float32(127))
    assert s[0] == floor and s[1] == floor and not q[0].any()
    assert q[1, 5] == 0  # 1e-12 / (1e-8/127) = 0.0127 -> 0


def _division_traps(n_amax=400):
    """bf16 pairs (amax, x) for which rint(x / s) != rint(x * (1 / s)) in fp32, s = amax / 127."""
    out = []
    amaxs = np.unique(bf16_bits(torch.from_numpy(np.abs(RNG.standard_normal(n_amax)).astype(np.float32) * 4 + 0.1)))
    allx = np.arange(0, 0x7F80, dtype=np.uint16)
    fx = oracle.bf2f(allx)
    for a in amaxs:
        af = oracle.bf2f(np.array([a]))[0]
        s = np.float32(af) / np.float32(127)
        cand = fx[fx <= af]
        hx = allx[: cand.size]
        q_div = np.rint(cand / s)
        q_rcp = np.rint(cand * (np.float32(1) / s))
        bad = np.nonzero(q_div != q_rcp)[0]
        for i in bad[:2]:
            out.append((a, hx[i]))
        if len(out) >= 16:
            break
    return out


def test_quant_rows_true_division_traps():
    """Rows built around (amax, x) pairs where multiplying by the reciprocal rounds differently: the oracle must
    follow true division (tests/test_int8_gemm.py:37 notes the 1-ulp difference)."""
    traps = _division_traps()
    assert len(traps) >= 4, "no trap pairs found"
    x = np.zeros((len(traps), 64), np.uint16)
    for r, (a, v) in enumerate(traps):
        x[r, 0] = a
        x[r, 1] = v
        x[r, 2] = v | 0x8000
    q, s = oracle.quant_rows(x)
    xf = oracle.bf2f(x)
    expect = np.clip(np.rint(xf / s[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(q, expect)
    wrong = np.clip(np.rint(xf * (np.float32(1) / s[:, None])), -127, 127).astype(np.int8)
    assert not np.array_equal(q, wrong)


def test_quant_rows_matches_reference_expression():
    """tests/test_int8_gemm.py:35-38 (ref_quant), evaluated by torch on the CPU."""
    x = rand_bf16((37, 1152)) * 1
    x = bf16_bits(from_bits(x).float() * torch.rand(37, 1, generator=torch.Generator().manual_seed(3)) * 4)
    x[0, 3] = bf16_bits(torch.tensor([37.0]))[0]
    q, s = oracle.quant_rows(x)
    xt = from_bits(x).float()
    a = xt.abs().amax(-1).clamp_min(1e-8)
    rs = a / torch.full_like(a, 127.0)
    rq = torch.round(xt / rs[:, None]).clamp(-127, 127).to(torch.int8)
    assert np.array_equal(q, rq.numpy()) and np.array_equal(s, rs.numpy())
    # dequantization error bound and full range use
    xf = oracle.bf2f(x)
    assert np.all(np.abs(q * s[:, None] - xf) <= s[:, None] * 0.5 * (1 + 1e-5))
    assert np.all(np.abs(q).max(1) == 127)


def test_quant_groups_is_quant_rows_per_group():
    x = rand_bf16((5, 256), 3.0)
    q, sT = oracle.quant_groups(x)
    assert sT.shape == (4, 5)
    for g in range(4):
        qg, sg = oracle.quant_rows(x[:, g * 64:(g + 1) * 64])
        assert np.array_equal(q[:, g * 64:(g + 1) * 64], qg) and np.array_equal(sT[g], sg)


# ------------------------------------------------------------------------------------------------ W8A8
def test_gemm_i8_i32_is_exact_integer_product():
    A = RNG.integers(-127, 128, (13, 200), dtype=np.int8)
    B = RNG.integers(-127, 128, (29, 200), dtype=np.int8)
    C = oracle.gemm_i8_i32(A, B)
    assert C.shape == (13, 29)
    assert np.array_equal(C, A.astype(np.int64) @ B.astype(np.int64).T)
    # extreme accumulators at the largest K of the workloads
    A = np.full((2, 8192), 127, np.int8)
    A[1] = -127
    B = np.full((3, 8192), 127, np.int8)
    C = oracle.gemm_i8_i32(A, B)
    assert C[0, 0] == 127 * 127 * 8192 and C[1, 2] == -127 * 127 * 8192


def test_gemm_epilogue_power_of_two_closed_form():
    """sx, sw powers of two and no bias: y = bf16(acc * 2^a * 2^b) exactly, per row / per column."""
    C = RNG.integers(-(1 << 20), 1 << 20, (6, 10), dtype=np.int32)
    sx = (2.0 ** RNG.integers(-12, 3, 6)).astype(np.float32)
    sw = (2.0 ** RNG.integers(-12, 3, 10)).astype(np.float32)
    y = oracle.gemm_i8_epilogue(C, sx, sw)
    exact = torch.from_numpy(C.astype(np.float64) * sx[:, None].astype(np.float64) * sw[None, :].astype(np.float64))
    assert np.array_equal(y, bf16_bits(exact.float()))


def test_gemm_i8_matches_reference_expression():
    """tests/test_int8_gemm.py:158-172: (xq.double() @ wq.double().t()).float() * sx[:, None] * sw[None, :] + b,
    then GELU (<= 1 bf16 ulp of F.gelu tanh, one fp32 ulp of the input where the formula cancels) or not
    (bit-exact)."""
    M, K, N = 17, 320, 24
    x = rand_bf16((M, K))
    w = rand_bf16((N, K), 0.02)
    b = rand_bf16((N,))
    xq, sx = oracle.quant_rows(x)
    wq, sw = oracle.quant_rows(w)
    acc = torch.from_numpy(xq).double() @ torch.from_numpy(wq).double().t()
    r = acc.float() * torch.from_numpy(sx)[:, None] * torch.from_numpy(sw)[None, :] + from_bits(b).float()
    y = oracle.gemm_i8(xq, sx, wq, sw, b)
    assert np.array_equal(y, bf16_bits(r))
    yg = oracle.gemm_i8(xq, sx, wq, sw, b, gelu=True)
    assert_gelu_close(yg, r)
    # a bias added before the scales, or a transposed weight, would not match
    assert not np.array_equal(y, oracle.gemm_i8(xq, sx, wq, sw, None))


def test_gemm_i8_grouped_close_to_fp64():
    """Grouped fold vs the fp64 per-group sum of tests/test_int8_gemm.py:81-104 (its tolerance rule)."""
    M, K, N = 9, 256, 16
    x = rand_bf16((M, K))
    x[:, 5] = bf16_bits(from_bits(x[:, 5]).float() * 30)
    w = rand_bf16((N, K), 0.02)
    xq, sxT = oracle.quant_groups(x)
    wq, sw = oracle.quant_rows(w)
    y = oracle.gemm_i8_grouped(xq, sxT, wq, sw)
    r = np.zeros((M, N))
    for g in range(K // 64):
        part = xq[:, g * 64:(g + 1) * 64].astype(np.float64) @ wq[:, g * 64:(g + 1) * 64].astype(np.float64).T
        r += part * sxT[g].astype(np.float64)[:, None]
    r *= sw.astype(np.float64)[None, :]
    e_ours = np.linalg.norm(oracle.bf2f(y) - r) / np.linalg.norm(r)
    e_round = np.linalg.norm(oracle.bf2f(bf16_bits(torch.from_numpy(r).float())) - r) / np.linalg.norm(r)
    assert e_ours <= 1.05 * e_round + 1e-6


def test_gemm_i8_grouped_rounding_points():
    """The grouped fold's operation sequence on constructed operands whose expected bits are derived by hand
    (tests/rounding_cases.py): fma per group in group order in an fp32 accumulator, then fl(fl(facc sw) + b). The
    slips each case is built to catch are evaluated here too, with separately rounded fp32 numpy arithmetic, to show
    that they give other bits."""
    xq, sxT, wq, sw, b, expect = rounding_cases.grouped_fold_case()
    y = oracle.gemm_i8_grouped(xq, sxT, wq, sw, b)
    for (m, n), bits in expect.items():
        assert int(y[m, n]) == bits, (m, n, hex(int(y[m, n])))
    f = np.float32
    part = [f(int(xq[0, 64 * g])) for g in range(3)]
    unfused = f(0)
    for g in range(3):  # product rounded before the add
        unfused = f(f(part[g] * sxT[g, 0]) + unfused)
    backwards = f(0)
    for g in (2, 1, 0):  # fma emulated exactly in fp64: every product here has at most 26 significant bits
        backwards = f(np.float64(part[g]) * np.float64(sxT[g, 0]) + np.float64(backwards))
    assert unfused == 0 and backwards == 0 and expect[0, 0] != 0
    wide = sum(np.float64(int(xq[1, 64 * g])) * np.float64(sxT[g, 1]) for g in range(3))
    assert wide == 2.0 ** -24 and expect[1, 0] == 0
    fused = np.float64(f(1 + 2.0 ** -23)) * np.float64(sw[1]) - 1.0  # fma(facc, sw, b): one rounding
    assert int(bf16_bits(torch.tensor([fused], dtype=torch.float32))[0]) == 0x3380 and expect[2, 1] == 0


def test_gemm_i8_epilogue_rounding_points():
    """Per-token epilogue on constructed operands (tests/rounding_cases.py): y = bf16(fl(fl(fl(acc sx) sw) + b)),
    with the expected bits derived by hand; fl(sx sw) first, or an fma of the last two operations, gives other bits
    (shown with separately rounded fp32 numpy arithmetic)."""
    xq, sx, wq, sw, b, expect = rounding_cases.per_token_epilogue_case()
    y = oracle.gemm_i8(xq, sx, wq, sw, b)
    for (m, n), bits in expect.items():
        assert int(y[m, n]) == bits, (m, n, hex(int(y[m, n])))
    f = np.float32
    assert f(f(f(3) * f(sx[0] * sw[0])) - f(3)) == f(3 * 2.0 ** -22)  # the other association: 0x3540
    assert np.float64(sx[1]) * np.float64(sw[1]) - 1.0 == 2.0 ** -24 - 2.0 ** -47  # what an fma would keep


# ------------------------------------------------------------------------------------------------ GEMVs
def test_gemv_one_hot_rows_closed_form():
    """W[n] = q_n e_{k_n} with N != K: y[b, n] = bf16(q_n x[b, k_n] 2^e_n) exactly; a transposed W or a wrong
    scale index cannot match."""
    N, K, B = 12, 64, 3
    kn = RNG.integers(0, K, N)
    qn = RNG.integers(-127, 128, N)
    W = np.zeros((N, K), np.int8)
    W[np.arange(N), kn] = qn
    sc = (2.0 ** RNG.integers(-10, 0, N)).astype(np.float32)
    x = rand_bf16((B, K))
    y = oracle.gemv(W, sc, x)
    exact = qn[None, :] * oracle.bf2f(x)[:, kn].astype(np.float64) * sc[None, :]
    assert np.array_equal(y, bf16_bits(torch.from_numpy(exact).float()))


def test_gemv_matches_fp64_and_reference_expression():
    N, K, B = 48, 512, 4
    W = RNG.integers(-127, 128, (N, K), dtype=np.int8)
    sc = (np.abs(RNG.standard_normal(N)) * 0.01 + 1e-3).astype(np.float32)
    x = rand_bf16((B, K))
    y = oracle.gemv(W, sc, x)
    exact = (oracle.bf2f(x).astype(np.float64) @ W.astype(np.float64).T) * sc[None, :]
    assert ulps(y, bf16_bits(torch.from_numpy(exact).float())) <= 1
    # tests/test_kernels.py:137: F.linear(x.float(), Wq.float() * scale[:, None]).to(bf16), tolerance :29-34
    ref = F.linear(from_bits(x).float(), torch.from_numpy(W).float() * torch.from_numpy(sc)[:, None])
    err = (from_bits(y).float() - ref).abs().max().item()
    assert err <= 2e-2 * max(ref.abs().max().item(), 1.0)
    # bf16 weights, no scale
    Wb = rand_bf16((N, K), 0.02)
    yb = oracle.gemv(Wb, None, x)
    exact = oracle.bf2f(x).astype(np.float64) @ oracle.bf2f(Wb).astype(np.float64).T
    assert ulps(yb, bf16_bits(torch.from_numpy(exact).float())) <= 1


def test_silu_mul_matches_torch_expression():
    g = rand_bf16((3, 2 * 300), 3.0)
    y = oracle.silu_mul(g)
    gt = from_bits(g)
    a, u = gt[:, :300].float(), gt[:, 300:].float()
    ref = (F.silu(a).to(torch.bfloat16).float() * u).to(torch.bfloat16)
    assert ulps(y, bf16_bits(ref.float())) <= 1


def test_swiglu_is_gemv_then_silu_mul():
    """gemv_epi(0) == gemv + silu_mul (the reference's definition, tests/test_kernels.py:153-186)."""
    S, K, B = 40, 256, 2
    W = RNG.integers(-127, 128, (2 * S, K), dtype=np.int8)
    sc = (np.abs(RNG.standard_normal(2 * S)) * 0.01 + 1e-3).astype(np.float32)
    x = rand_bf16((B, K))
    assert np.array_equal(oracle.gemv_swiglu(W, sc, x), oracle.silu_mul(oracle.gemv(W, sc, x)))


def test_residual_is_gemv_then_add():
    N, K, B = 24, 128, 3
    W = RNG.integers(-127, 128, (N, K), dtype=np.int8)
    sc = (np.abs(RNG.standard_normal(N)) * 0.01).astype(np.float32)
    x, h = rand_bf16((B, K)), rand_bf16((B, N))
    y = oracle.gemv(W, sc, x)
    hn = oracle.gemv_residual(W, sc, x, h)
    ref = (from_bits(h).float() + from_bits(y).float()).to(torch.bfloat16)
    assert np.array_equal(hn, bf16_bits(ref.float()))
    assert np.array_equal(oracle.gemv_residual(W, sc, x, np.zeros_like(h)), y)


# ------------------------------------------------------------------------------------------------ INT4
def pack_ref_int4(q):
    """src/lfm2opt/quant.py:37-38 packing, q in [-8, 7] -> uint8 [N, K/2] (element 2j low nibble, stored q + 8)."""
    u = (q + 8).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def test_gemv_w4_nibble_order_known_answer():
    N, K, group = 2, 64, 32
    Wp = np.full((N, K // 2), 0x88, np.uint8)  # all q = 0
    Wp[0, 0] = 0x21  # k0: nibble 1 -> q - 8 = -7; k1: nibble 2 -> -6
    S = np.ones((N, K // group), np.float32)
    S[0, 0] = 0.5
    for k, expect in ((0, -3.5), (1, -3.0), (2, 0.0)):
        x = np.zeros((1, K), np.uint16)
        x[0, k] = 0x3F80  # 1.0
        y = oracle.gemv_w4(Wp, S, x)
        assert oracle.bf2f(y)[0, 0] == expect and y[0, 1] == 0


def test_gemv_w4_matches_dequantized_fp64():
    N, K, group = 16, 512, 128
    q = RNG.integers(-8, 8, (N, K))
    S = (np.abs(RNG.standard_normal((N, K // group))) * 0.02 + 1e-3).astype(np.float32)
    Wp = pack_ref_int4(q)
    x = rand_bf16((1, K))
    w = q.astype(np.float64) * np.repeat(S.astype(np.float64), group, axis=1)
    exact = oracle.bf2f(x).astype(np.float64) @ w.T
    assert ulps(oracle.gemv_w4(Wp, S, x), bf16_bits(torch.from_numpy(exact).float())) <= 1


def pack_w4z(q, z):
    """q [N, K] in [0, 15] -> int32 [N, K/8] (nibble i of word w = k 8w + i); z [N, G] -> int32 [N, ceil(G/8)]."""
    N, K = q.shape
    qw = np.zeros((N, K // 8), np.uint32)
    for i in range(8):
        qw |= (q[:, i::8].astype(np.uint32) & 15) << (4 * i)
    G = z.shape[1]
    zw = np.zeros((N, (G + 7) // 8), np.uint32)
    for g in range(G):
        zw[:, g // 8] |= (z[:, g].astype(np.uint32) & 15) << (4 * (g % 8))
    return qw.view(np.int32), zw.view(np.int32)


def test_gemv_w4z_reduces_to_reference_format():
    """Z = 8 and fp16-exact scales: the zero-point format is the reference format (same bytes, read as int32)."""
    N, K, group = 16, 512, 128
    q = RNG.integers(-8, 8, (N, K))
    S16 = (np.abs(RNG.standard_normal((N, K // group))) * 0.02 + 1e-3).astype(np.float16)
    Wp = pack_ref_int4(q)
    Wq, Z = pack_w4z(q + 8, np.full((N, K // group), 8))
    assert np.array_equal(Wq.view(np.uint8).reshape(N, K // 2), Wp)  # identical bytes
    x = rand_bf16((2, K))
    y_ref = oracle.gemv_w4(Wp, S16.astype(np.float32), x)
    y_z = oracle.gemv_w4z(Wq, S16, Z, x, group)
    assert np.array_equal(y_ref, y_z)


def test_gemv_w4z_zero_points_and_swiglu():
    N, K, group = 8, 256, 128
    q = RNG.integers(0, 16, (N, K))
    z = RNG.integers(0, 16, (N, K // group))
    S16 = (np.abs(RNG.standard_normal((N, K // group))) * 0.02 + 1e-3).astype(np.float16)
    Wq, Z = pack_w4z(q, z)
    x = rand_bf16((3, K))
    w = (q - np.repeat(z, group, axis=1)).astype(np.float64) * np.repeat(S16.astype(np.float64), group, axis=1)
    exact = oracle.bf2f(x).astype(np.float64) @ w.T
    y = oracle.gemv_w4z(Wq, S16, Z, x, group)
    assert ulps(y, bf16_bits(torch.from_numpy(exact).float())) <= 1
    ys = oracle.gemv_w4z(Wq, S16, Z, x, group, swiglu=True)
    assert np.array_equal(ys, oracle.silu_mul(y))


# ------------------------------------------------------------------------------------------------ INT8 producers
def test_add_rmsnorm_against_torch_fp64():
    """h = bf16(h + y) exactly as torch's bf16 add; x within 1 bf16 ulp of bf16(w * bf16(F.rms_norm(h) in fp64))."""
    rows, H, eps = 37, 512, 1e-5
    h, y = rand_bf16((rows, H), 2.0), rand_bf16((rows, H))
    w = bf16_bits(torch.from_numpy(RNG.random(H).astype(np.float32) + 0.5))
    hn, x = oracle.add_rmsnorm(h, y, w, eps)
    assert np.array_equal(hn, bf16_bits((from_bits(h).float() + from_bits(y).float())))
    hd = from_bits(hn).double()
    n = F.rms_norm(hd, (H,), eps=eps).to(torch.bfloat16).float()
    ref = bf16_bits(from_bits(w).float()[None, :] * n)
    assert ulps(x, ref) <= 1 and (x != ref).mean() < 0.01
    # no residual input: h is left as it is
    hn2, x2 = oracle.add_rmsnorm(hn, None, w, eps)
    assert np.array_equal(hn2, hn) and np.array_equal(x2, x)


def test_add_rmsnorm_constant_rows_closed_form():
    """A constant row c (|c| >= 1, eps = 1e-5) normalizes to exactly sign(c), so x = sign(c) * w bit for bit."""
    H = 256
    c = np.array([1.0, -3.0, 40.0, -1.5], np.float32)
    h = bf16_bits(torch.from_numpy(np.repeat(c[:, None], H, 1)))
    w = rand_bf16((H,))
    _, x = oracle.add_rmsnorm(h, None, w, 1e-5)
    wf = oracle.bf2f(w)
    for r in range(4):
        assert np.array_equal(x[r], oracle.f2bf(np.sign(c[r]) * wf))


def test_add_layernorm_against_torch_fp64():
    rows, D, eps = 29, 1152, 1e-6
    h, y = rand_bf16((rows, D), 3.0), rand_bf16((rows, D))
    h[:, :7] = bf16_bits(from_bits(h[:, :7]).float() + 5.0)  # a mean far from zero
    w = bf16_bits(torch.from_numpy(RNG.random(D).astype(np.float32) + 0.5))
    b = rand_bf16((D,))
    hn, x = oracle.add_layernorm(h, y, w, b, eps)
    assert np.array_equal(hn, bf16_bits((from_bits(h).float() + from_bits(y).float())))
    ref = F.layer_norm(from_bits(hn).double(), (D,), from_bits(w).double(), from_bits(b).double(), eps)
    assert ulps(x, bf16_bits(ref.float())) <= 1


def test_add_layernorm_two_level_rows_closed_form():
    """Rows alternating a and -a: mean 0, var a^2, so (h - mean) * rstd = +-1 up to eps and x = bf16(+-w + b)."""
    D = 128
    a = np.array([2.0, 0.5, 8.0], np.float32)
    sign = np.where(np.arange(D) % 2 == 0, 1.0, -1.0).astype(np.float32)
    h = bf16_bits(torch.from_numpy(a[:, None] * sign[None, :]))
    w = rand_bf16((D,))
    b = rand_bf16((D,))
    _, x = oracle.add_layernorm(h, None, w, b, 1e-9)
    wf, bf = oracle.bf2f(w), oracle.bf2f(b)
    for r in range(3):
        assert np.array_equal(x[r], oracle.f2bf(sign * wf + bf))


# ------------------------------------------------------------------------------------------------ W8A16
def test_gemm_w8_against_torch_fp64():
    """acc in fp64 rounded once, then * sw + b: within 1 bf16 ulp of torch's fp64 (x @ w^T) * sw + b; bit-exact when
    sw and x are powers of two (every intermediate exact)."""
    M, K, N = 9, 384, 20
    x = rand_bf16((M, K))
    W = RNG.integers(-127, 128, (N, K), dtype=np.int8)
    sw = (np.abs(RNG.standard_normal(N)) * 0.01 + 1e-3).astype(np.float32)
    b = rand_bf16((N,))
    y = oracle.gemm_w8(x, W, sw, b)
    r = (from_bits(x).double() @ torch.from_numpy(W).double().t()) * torch.from_numpy(sw).double() + from_bits(b).double()
    assert ulps(y, bf16_bits(r.float())) <= 1
    x2 = bf16_bits(torch.from_numpy((2.0 ** RNG.integers(-3, 3, (M, K))).astype(np.float32)))
    sw2 = (2.0 ** RNG.integers(-10, -4, N)).astype(np.float32)
    y2 = oracle.gemm_w8(x2, W, sw2)
    r2 = (from_bits(x2).double() @ torch.from_numpy(W).double().t()) * torch.from_numpy(sw2).double()
    assert np.array_equal(y2, bf16_bits(r2.float()))
    yg = oracle.gemm_w8(x, W, sw, b, gelu=True)
    assert_gelu_close(yg, r.float())
