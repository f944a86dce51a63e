"""INT4 weight-only GEMVs on the GPU (through the C ABI via lfm2opt.kernels.ext()) against the CPU oracle.

Parity bar: bf16 outputs within max |err| / max |ref| <= 1e-2 (mean abs err and max bf16 ulps reported), as for the
INT8 GEMVs; the fused SwiGLU and residual epilogues bit-identical to the plain GEMV followed by the separate op; the
reference format bit-identical to the GPTQ-style format when the zero points are 8 and the scales are fp16-exact
(the same weights in the two layouts). Shapes cover batch 1 (VALU kernel), 2..16 (matrix-core kernel), batches above
16 (chunks), group sizes below 128 with batch > 1 (per-row fallback), K below one wavefront's 2048 weights, and the
LFM2 decode shapes.
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN
from gpu_util import assert_close_bf16, dev, dev_bf16, host_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import ext

    return ext()


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


def pack_ref(q):
    u = (q + 8).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def pack_nibbles(v):
    R, C = v.shape
    pad = np.zeros((R, -(-C // 8) * 8), np.uint32)
    pad[:, :C] = v
    w = np.zeros((R, pad.shape[1] // 8), np.uint32)
    for i in range(8):
        w |= pad[:, i::8] << np.uint32(4 * i)
    return w.view(np.int32)


def gen_ref(seed, B, R, K, group):
    r = np.random.default_rng(seed)
    q = r.integers(-8, 8, (R, K))
    S = (np.abs(r.standard_normal((R, K // group))) * 0.02 + 1e-3).astype(np.float32)
    x = oracle.f2bf(r.standard_normal((B, K)).astype(np.float32))
    return pack_ref(q), S, x


def gen_zp(seed, B, R, K, group):
    r = np.random.default_rng(seed)
    q = r.integers(0, 16, (R, K))
    z = r.integers(0, 16, (R, K // group))
    S = (np.abs(r.standard_normal((R, K // group))) * 0.02 + 1e-3).astype(np.float16)
    x = oracle.f2bf(r.standard_normal((B, K)).astype(np.float32))
    return pack_nibbles(q), S, pack_nibbles(z), x


def run_ref(E, Wp, S, x, epi=0, h=None):
    B, K = x.shape
    N = Wp.shape[0] // (2 if epi == 1 else 1)
    y = dev_bf16(h) if h is not None else torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv_w4(dev(Wp), dev(S), dev_bf16(x), y, 0, epi)
    return host_bits(y)


def run_zp(E, Wq, S, Z, x, epi=0, h=None):
    B, K = x.shape
    N = Wq.shape[0] // (2 if epi == 1 else 1)
    y = dev_bf16(h) if h is not None else torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv_w4z(dev(Wq), dev(S), dev(Z), dev_bf16(x), y, epi)
    return host_bits(y)


# ------------------------------------------------------------------------------------------------ fixtures
@pytest.mark.parametrize("name", ["gemv_w4_b1_n80_k1024_g128", "gemv_w4_b4_n48_k2048_g128", "gemv_w4_b2_n40_k512_g64"])
def test_gemv_w4_fixture(E, name):
    d = load(name)
    assert_close_bf16(run_ref(E, d["Wp"], d["S"], d["x"]), d["y"], what=name)


@pytest.mark.parametrize("name,epi", [("gemv_w4z_b1_r64_k2048_g128", 0), ("gemv_w4z_b8_r96_k1024_g128_swiglu", 1)])
def test_gemv_w4z_fixture(E, name, epi):
    d = load(name)
    out = run_zp(E, d["Wq"], d["S"].view(np.float16), d["Z"], d["x"], epi)
    assert_close_bf16(out, d["y"], what=name)


# ------------------------------------------------------------------------------------------------ vs oracle
@pytest.mark.parametrize("B", [1, 2, 5, 8, 16, 20])
@pytest.mark.parametrize("N,K,group", [(300, 2048, 128), (257, 8192, 128), (64, 1536, 128), (136, 1152, 128),
                                       (72, 96, 32)])
def test_gemv_w4_vs_oracle(E, B, N, K, group):
    Wp, S, x = gen_ref(N + K + B, B, N, K, group)
    assert_close_bf16(run_ref(E, Wp, S, x), oracle.gemv_w4(Wp, S, x), what=f"gemv_w4 B={B} [{N}x{K}] g{group}")


@pytest.mark.parametrize("shape", ["1,1,1", "1,1,4", "1,2,2", "1,2,4", "1,2,16", "1,4,2", "1,4,4", "2,1,1", "2,1,4",
                                   "2,1,16"])
def test_gemv_w4_mfma_launch_shapes(E, tune, shape):
    """Every batch-2..16 launch shape of the matrix-core INT4 kernel (k-parts KS, row tiles RT, wavefronts NWK,
    forced through the LFM2Q_W4_MFMA knob), with a trailing half block (K = 1152) and N not a multiple of the tile
    rows, in both weight formats and with every epilogue:
      plain       against the oracle;
      SwiGLU      (W = w1|w3, 2 N rows; RT = 2 puts two w1 and two w3 tiles in one workgroup) against the oracle, and
                  bit-identical to the plain GEMV + silu_mul under the same shape (RT = 4 does not apply to SwiGLU,
                  whose shape then differs from the plain call's, so only the oracle bar holds there);
      residual    bit-identical to the plain GEMV + the bf16 add."""
    tune("LFM2Q_W4_MFMA", shape)
    N, K, group = 300, 1152, 128
    same_shape = shape.split(",")[1] != "4"
    for B in (3, 8) if shape.startswith("2") else (3, 13):
        h0 = oracle.f2bf(np.random.default_rng(B).standard_normal((B, N)).astype(np.float32) * 4)
        # reference format
        Wp, S, x = gen_ref(B + 7, B, N, K, group)
        y = run_ref(E, Wp, S, x)
        assert_close_bf16(y, oracle.gemv_w4(Wp, S, x), what=f"gemv_w4 shape {shape} B={B}")
        assert np.array_equal(run_ref(E, Wp, S, x, 2, h0), oracle.f2bf(oracle.bf2f(h0) + oracle.bf2f(y)))
        W2, S2, x2 = gen_ref(B + 8, B, 2 * N, K, group)
        sw = run_ref(E, W2, S2, x2, 1)
        plain2 = run_ref(E, W2, S2, x2)
        assert_close_bf16(sw, oracle.silu_mul(oracle.gemv_w4(W2, S2, x2)), what=f"gemv_w4 swiglu shape {shape} B={B}")
        if same_shape:
            assert np.array_equal(sw, oracle.silu_mul(plain2)), f"swiglu != gemv + silu_mul, shape {shape} B={B}"
        # GPTQ-style format
        Wq, Sz, Z, xz = gen_zp(B + 9, B, N, K, group)
        yz = run_zp(E, Wq, Sz, Z, xz)
        assert_close_bf16(yz, oracle.gemv_w4z(Wq, Sz, Z, xz, group), what=f"gemv_w4z shape {shape} B={B}")
        assert np.array_equal(run_zp(E, Wq, Sz, Z, xz, 2, h0), oracle.f2bf(oracle.bf2f(h0) + oracle.bf2f(yz)))
        Wq2, Sz2, Z2, xz2 = gen_zp(B + 10, B, 2 * N, K, group)
        swz = run_zp(E, Wq2, Sz2, Z2, xz2, 1)
        assert_close_bf16(swz, oracle.gemv_w4z(Wq2, Sz2, Z2, xz2, group, swiglu=True),
                          what=f"gemv_w4z swiglu shape {shape} B={B}")
        if same_shape:
            assert np.array_equal(swz, oracle.silu_mul(run_zp(E, Wq2, Sz2, Z2, xz2)))


@pytest.mark.parametrize("B", [2, 8, 16])
@pytest.mark.parametrize("fmt", [0, 1])
def test_gemv_w4_swiglu_two_row_tiles_at_w13_shape(E, B, fmt):
    """w1|w3 at its decode shape (16384 x 2048) at batches 2-16: the automatic launch takes two row tiles per
    workgroup (6144+ weight rows), the path config 5's batch-8 decode step runs. Against the oracle on 64 sampled
    output rows, and bit-identical to the plain GEMV + silu_mul."""
    Sn, K, group = 8192, 2048, 128
    r = np.random.default_rng(90 + B + fmt)
    rows = np.sort(r.permutation(Sn)[:64])
    wr = np.concatenate([rows, Sn + rows])
    if fmt == 0:
        Wp, S, x = gen_ref(91 + B, B, 2 * Sn, K, group)
        fused, plain = run_ref(E, Wp, S, x, 1), run_ref(E, Wp, S, x, 0)
        ref = oracle.silu_mul(oracle.gemv_w4(Wp[wr], S[wr], x))
    else:
        Wq, S, Z, x = gen_zp(92 + B, B, 2 * Sn, K, group)
        fused, plain = run_zp(E, Wq, S, Z, x, 1), run_zp(E, Wq, S, Z, x, 0)
        ref = oracle.gemv_w4z(Wq[wr], S[wr], Z[wr], x, group, swiglu=True)
    assert_close_bf16(fused[:, rows], ref, what=f"w4 fmt {fmt} w1|w3 swiglu B={B} sampled rows")
    assert np.array_equal(fused, oracle.silu_mul(plain))


@pytest.mark.parametrize("B", [1, 4, 8, 16])
def test_gemv_w4z_residual_vs_oracle_and_add(E, B):
    """The GPTQ-style residual epilogue at the w2 and out-proj shapes: against the oracle's GEMV + bf16 add on 64
    sampled rows, and bit-identical to the library's plain GEMV + the bf16 add."""
    for N, K in ((2048, 8192), (2048, 2048)):
        Wq, S, Z, x = gen_zp(95 + B + K, B, N, K, 128)
        h0 = oracle.f2bf(np.random.default_rng(B + K).standard_normal((B, N)).astype(np.float32) * 4)
        fused, plain = run_zp(E, Wq, S, Z, x, 2, h0), run_zp(E, Wq, S, Z, x, 0)
        assert np.array_equal(fused, oracle.f2bf(oracle.bf2f(h0) + oracle.bf2f(plain)))
        rows = np.sort(np.random.default_rng(K).permutation(N)[:64])
        ref = oracle.f2bf(oracle.bf2f(h0[:, rows]) + oracle.bf2f(oracle.gemv_w4z(Wq[rows], S[rows], Z[rows], x, 128)))
        assert_close_bf16(fused[:, rows], ref, what=f"gemv_w4z residual B={B} [{N}x{K}] sampled rows")


@pytest.mark.parametrize("B", [1, 3, 8, 17])
@pytest.mark.parametrize("N,K,group", [(200, 2048, 128), (96, 8192, 256), (40, 1024, 64)])
def test_gemv_w4z_vs_oracle(E, B, N, K, group):
    Wq, S, Z, x = gen_zp(N + K + B + 1, B, N, K, group)
    assert_close_bf16(run_zp(E, Wq, S, Z, x), oracle.gemv_w4z(Wq, S, Z, x, group),
                      what=f"gemv_w4z B={B} [{N}x{K}] g{group}")


@pytest.mark.parametrize("B", [1, 8])
def test_gemv_w4z_swiglu_vs_oracle(E, B):
    Wq, S, Z, x = gen_zp(5 + B, B, 2 * 1000, 2048, 128)
    assert_close_bf16(run_zp(E, Wq, S, Z, x, 1), oracle.gemv_w4z(Wq, S, Z, x, 128, swiglu=True),
                      what=f"gemv_w4z swiglu B={B}")


# ------------------------------------------------------------------------------------------------ invariants
@pytest.mark.parametrize("B", [1, 4, 8, 16])
def test_reference_format_equals_zero_point_format_with_z8(E, B):
    """The same weights as uint8 [N, K/2] (zero point 8, fp32 scales) and as int32 [N, K/8] (zero points 8, fp16
    scales holding the same values) give bit-identical results."""
    N, K, group = 520, 2048, 128
    Wp, S, x = gen_ref(40 + B, B, N, K, group)
    S16 = S.astype(np.float16)
    Z = pack_nibbles(np.full((N, K // group), 8))
    a = run_ref(E, Wp, S16.astype(np.float32), x)
    b = run_zp(E, Wp.view("<i4"), S16, Z, x)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("B", [1, 2, 8, 16])
@pytest.mark.parametrize("fmt", [0, 1])
def test_swiglu_bit_identical_to_gemv_then_silu_mul(E, B, fmt):
    Sn, K, group = 1024, 2048, 128
    if fmt == 0:
        Wp, S, x = gen_ref(60 + B, B, 2 * Sn, K, group)
        fused = run_ref(E, Wp, S, x, 1)
        plain = run_ref(E, Wp, S, x, 0)
    else:
        Wq, S, Z, x = gen_zp(70 + B, B, 2 * Sn, K, group)
        fused = run_zp(E, Wq, S, Z, x, 1)
        plain = run_zp(E, Wq, S, Z, x, 0)
    g = dev_bf16(plain)
    y = torch.empty(B, Sn, device="cuda", dtype=torch.bfloat16)
    E.silu_mul(g, y)
    assert np.array_equal(fused, host_bits(y))


@pytest.mark.parametrize("B", [1, 8])
def test_residual_bit_identical_to_gemv_then_add(E, B):
    N, K, group = 2048, 8192, 128
    Wp, S, x = gen_ref(80 + B, B, N, K, group)
    h = oracle.f2bf(np.random.default_rng(3).standard_normal((B, N)).astype(np.float32) * 4)
    fused = run_ref(E, Wp, S, x, 2, h)
    plain = run_ref(E, Wp, S, x, 0)
    ref = oracle.f2bf(oracle.bf2f(h) + oracle.bf2f(plain))
    assert np.array_equal(fused, ref)


# ------------------------------------------------------------------------------------------------ decode shapes
@pytest.mark.parametrize("N,K", [(3072, 2048), (6144, 2048), (2048, 8192), (65536, 2048)])
@pytest.mark.parametrize("B", [1, 8])
def test_gemv_w4z_decode_shapes(E, N, K, B):
    """LFM2 decode shapes in the GPTQ-style format: against torch's fp32 dequant-matmul on the GPU
    (tests/test_kernels.py:150) and, on 48 sampled rows, against the CPU oracle."""
    from lfm2opt.quant import dequantize_int4_zp

    Wq, S, Z, x = gen_zp(N + K + B, B, N, K, 128)
    Wq_d, S_d, Z_d, x_d = dev(Wq), dev(S), dev(Z), dev_bf16(x)
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv_w4z(Wq_d, S_d, Z_d, x_d, y)
    ref = (x_d.float() @ dequantize_int4_zp(Wq_d, S_d, Z_d).t()).to(torch.bfloat16)
    assert_close_bf16(host_bits(y), host_bits(ref), what=f"gemv_w4z B={B} [{N}x{K}] vs torch fp32")
    rows = np.sort(np.random.default_rng(4).permutation(N)[:48])
    ro = oracle.gemv_w4z(Wq[rows], S[rows], Z[rows], x, 128)
    assert_close_bf16(host_bits(y)[:, rows], ro, what=f"gemv_w4z B={B} [{N}x{K}] sampled rows vs oracle")


# ------------------------------------------------------------------------------------------------ argument errors
def test_w4_argument_errors_raise_before_launch(E):
    Wp = torch.zeros(64, 256, device="cuda", dtype=torch.uint8)
    S = torch.ones(64, 4, device="cuda")
    x = torch.zeros(1, 512, device="cuda", dtype=torch.bfloat16)
    y = torch.zeros(1, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Wp: contiguous uint8"):
        E.gemv_w4(Wp.to(torch.int8), S, x, y)
    with pytest.raises(RuntimeError, match="S: contiguous fp32"):
        E.gemv_w4(Wp, S.half(), x, y)
    with pytest.raises(RuntimeError, match="group size must be a multiple of 32"):
        E.gemv_w4(Wp, torch.ones(64, 32, device="cuda"), x, y)
    with pytest.raises(RuntimeError, match="S must be"):
        E.gemv_w4(Wp, torch.ones(64, 3, device="cuda"), x, y)
    with pytest.raises(RuntimeError, match=r"x \[B, K\], y \[B, N\]"):
        E.gemv_w4(Wp, S, x, torch.zeros(1, 63, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="K <= 8192"):
        E.gemv_w4(torch.zeros(8, 8192, device="cuda", dtype=torch.uint8), torch.ones(8, 128, device="cuda"),
                  torch.zeros(1, 16384, device="cuda", dtype=torch.bfloat16),
                  torch.zeros(1, 8, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="qzeros"):
        E.gemv_w4z(torch.zeros(64, 64, device="cuda", dtype=torch.int32), S.half(),
                   torch.zeros(64, 2, device="cuda", dtype=torch.int32), x, y)
    torch.cuda.synchronize()


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("N,K,group", [(3001, 2048, 128), (130, 4096, 128), (257, 8192, 128), (77, 1024, 64)])
def test_one_shot_matches_persistent(E, tune, fmt, N, K, group):
    """Batch 1: the one-shot kernel (LFM2Q_W4_ONESHOT=1, the default below 32768 weight rows) and the persistent
    kernel (LFM2Q_W4_ONESHOT=0) give the same bits, plain, SwiGLU and residual, in both weight formats."""
    h0 = oracle.f2bf(np.random.default_rng(N).standard_normal((1, N)).astype(np.float32) * 4)
    if fmt == 0:
        Wp, S, x = gen_ref(N + K, 1, N, K, group)
        runs = lambda epi, h=None, n=N: run_ref(E, Wp[:n], S[:n], x, epi, h)  # noqa: E731
    else:
        Wq, S, Z, x = gen_zp(N + K + 1, 1, N, K, group)
        runs = lambda epi, h=None, n=N: run_zp(E, Wq[:n], S[:n], Z[:n], x, epi, h)  # noqa: E731
    res = {}
    for mode in ("1", "0"):
        tune("LFM2Q_W4_ONESHOT", mode)
        res[mode] = (runs(0), runs(1, n=2 * (N // 2)), runs(2, h0))
    for a, b in zip(res["1"], res["0"]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("N,K,group", [(2048, 2048, 128), (3074, 2048, 128), (1030, 8192, 128), (130, 4096, 128),
                                       (77, 1024, 64), (38, 3072, 128)])
def test_one_shot_shared_repack_matches_per_wavefront(E, tune, fmt, N, K, group):
    """Batch 1, one-shot kernel: the form whose workgroup repacks the activation row once into LDS
    (LFM2Q_GEMV_XS=1) gives the bits of the form where every wavefront repacks it (=0), plain, SwiGLU and residual,
    in both weight formats; N not a multiple of the workgroup's 8 rows (wavefronts past the end take part in the
    repack and store nothing) and K below a wavefront's 2048 CPL weights (chunks past K are zero)."""
    h0 = oracle.f2bf(np.random.default_rng(N + 1).standard_normal((1, N)).astype(np.float32) * 4)
    if fmt == 0:
        Wp, S, x = gen_ref(N + K + 2, 1, N, K, group)
        runs = lambda epi, h=None, n=N: run_ref(E, Wp[:n], S[:n], x, epi, h)  # noqa: E731
    else:
        Wq, S, Z, x = gen_zp(N + K + 3, 1, N, K, group)
        runs = lambda epi, h=None, n=N: run_zp(E, Wq[:n], S[:n], Z[:n], x, epi, h)  # noqa: E731
    tune("LFM2Q_W4_ONESHOT", 1)
    res = {}
    for mode in ("1", "0"):
        tune("LFM2Q_GEMV_XS", mode)
        res[mode] = (runs(0), runs(1, n=2 * (N // 2)), runs(2, h0))
    for a, b in zip(res["1"], res["0"]):
        assert np.array_equal(a, b)
