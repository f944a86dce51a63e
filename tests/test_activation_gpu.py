"""SiLU over its whole input domain, at each place the kernels evaluate it, and the GELU epilogue's far tails.

Every SiLU in the library takes a bf16 value (the SwiGLU gate g, rounded to bf16 as the reference rounds it,
kernels/lfm2_decode.cu:786-790 and :954-963) and rounds silu(g) to bf16, so the 65536 bf16 bit patterns -- zeros,
denormals, both infinities and NaNs included -- are its entire domain. With the up projection u = 1 every output is
bf16(silu(g)) exactly, and each is checked bit for bit against the oracle's g / (1 + expf(-g)) (the C library's
expf and an IEEE division), NaN against NaN. The gate values reach the kernels as the silu_mul / silu_mul_q input
itself, or through a GEMV whose weights select column 0 (x[:, 0] = 1, every other x and weight 0) so that the
accumulator is 1 and g is the row's scale (INT8, INT4) or weight (bf16).

The GELU epilogue's input is an fp32 GEMM value, not a bf16 one; its range [-10, 10] is swept densely by
tests/test_gemm_gpu.py, and here the tails past it (where tanh rounds to +-1, and past |v| ~ 7e12 where the cube
overflows) against the oracle's fp32 GELU."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import dev, dev_bf16, host_bits, ulp_dist

pytestmark = pytest.mark.gpu

ONE = 0x3F80  # bf16 1.0


@pytest.fixture(scope="module")
def D(cuda):
    from lfm2opt.kernels import ext

    return ext()


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import int8_ext

    return int8_ext()


def is_nan(h):
    return ((h & 0x7F80) == 0x7F80) & ((h & 0x7F) != 0)


gates = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)  # every bf16 bit pattern


def assert_same_bits(got, want, what, g=gates):
    """bit-identical, any NaN matching any NaN; the first differing gates are named."""
    got, want = np.asarray(got, np.uint16).ravel(), np.asarray(want, np.uint16).ravel()
    both = is_nan(got) & is_nan(want)
    bad = np.flatnonzero(np.where(both, False, got != want))
    msg = ", ".join(f"g={int(g[i]):#06x}: {int(got[i]):#06x} != {int(want[i]):#06x}" for i in bad[:6])
    assert bad.size == 0, f"{what}: {bad.size} outputs differ ({msg})"


def finite_gates():
    return gates[(gates & 0x7F80) != 0x7F80]


def want_silu(g):
    """bf16(silu(g)) for each gate, from the oracle's silu_mul with u = 1."""
    return oracle.silu_mul(np.concatenate([g, np.full_like(g, ONE)])[None, :])[0]


def test_silu_mul_every_bf16_input(D):
    g = np.concatenate([gates.reshape(8, 8192), np.full((8, 8192), ONE, np.uint16)], axis=1)
    y = torch.empty(8, 8192, device="cuda", dtype=torch.bfloat16)
    D.silu_mul(dev_bf16(g), y)
    assert_same_bits(host_bits(y).ravel(), want_silu(gates), "silu_mul")


@pytest.mark.parametrize("grouped", [False, True])
def test_silu_mul_q_every_bf16_input(E, grouped):
    """The fused SwiGLU + quantization producer's bf16 x (the row it quantizes)."""
    rows, I = 8, 8192
    g = np.concatenate([gates.reshape(rows, I), np.full((rows, I), ONE, np.uint16)], axis=1)
    x = torch.empty(rows, I, device="cuda", dtype=torch.bfloat16)
    q = torch.empty(rows, I, device="cuda", dtype=torch.int8)
    s = torch.empty((I // 64, rows) if grouped else (rows,), device="cuda", dtype=torch.float32)
    E.silu_mul_q(dev_bf16(g), q, s, x=x)
    assert_same_bits(host_bits(x).ravel(), want_silu(gates), f"silu_mul_q grouped={grouped}")


def summed(g):
    """the gate a dot product delivers: -0 plus the +0 products is +0."""
    return np.where(g == 0x8000, np.uint16(0), g)


def selector_x(B, K):
    x = torch.zeros(B, K, device="cuda", dtype=torch.bfloat16)
    x[:, 0] = 1.0
    return x


def gate_floats(g):
    return (g.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("B", [1, 4, 16])
def test_int8_swiglu_gemv_every_bf16_gate(D, B):
    """The INT8 fused SwiGLU GEMV (w1|w3 at K = 2048, the decode path's kernels for batch 1 and the matrix-core ones
    above it): g = bf16(1 x scale) runs over every bf16 pattern, u = 1."""
    S, K = gates.size, 2048
    W = torch.zeros(2 * S, K, device="cuda", dtype=torch.int8)
    W[:, 0] = 1
    sc = dev(np.concatenate([gate_floats(gates), np.ones(S, np.float32)]))
    y = torch.empty(B, S, device="cuda", dtype=torch.bfloat16)
    D.gemv_epi(0, W, sc, selector_x(B, K), y)
    want = want_silu(gates)
    for b in range(B):
        assert_same_bits(host_bits(y)[b], want, f"int8 swiglu gemv B={B} row {b}")


def test_bf16_swiglu_gemv_every_bf16_gate(D):
    """The bf16-weight fused SwiGLU GEMV: g = the row's weight at column 0. The gate -0 arrives as +0: the
    accumulator adds the row's other products (+0) to it, as the reference's dot product does."""
    S, K = gates.size, 2048
    W = torch.zeros(2 * S, K, device="cuda", dtype=torch.bfloat16)
    W[:S, 0] = dev_bf16(gates)
    W[S:, 0] = 1.0
    y = torch.empty(1, S, device="cuda", dtype=torch.bfloat16)
    D.gemv_epi(0, W, None, selector_x(1, K), y)
    assert_same_bits(host_bits(y)[0], want_silu(summed(gates)), "bf16 swiglu gemv")


@pytest.mark.parametrize("B", [1, 8])
def test_int4_swiglu_gemv_every_finite_bf16_gate(D, B):
    """The INT4 fused SwiGLU GEMV (reference format, group 128): weight 1 at column 0 (nibble 9), 0 elsewhere
    (nibble 8); g = bf16(group 0's scale). The finite gates only: with an inf or NaN scale the gate depends on where
    the dequantization applies the scale (inf x 0 is NaN), not on the SiLU. The gate -0 arrives as +0 (the other
    groups' +0 partial sums are added to it)."""
    g = finite_gates()
    S, K, group = g.size, 2048, 128
    Wp = torch.full((2 * S, K // 2), 0x88, device="cuda", dtype=torch.uint8)
    Wp[:, 0] = 0x89
    Sc = torch.ones(2 * S, K // group, device="cuda", dtype=torch.float32)
    Sc[:S, 0] = dev(gate_floats(g))
    y = torch.empty(B, S, device="cuda", dtype=torch.bfloat16)
    D.gemv_w4(Wp, Sc, selector_x(B, K), y, epi=1)
    want = want_silu(summed(g))
    for b in range(B):
        assert_same_bits(host_bits(y)[b], want, f"int4 swiglu gemv B={B} row {b}", g)


def test_gemm_gelu_epilogue_far_tails(E):
    """GELU on v = (1 x sx[m]) sw[n] + b[n] with |sx| log-spaced over [20, 1e37] (|v| >= 10): tanh(u) rounds to +-1
    in fp32 there, so the result is v on the positive side and -0 on the negative one, also past |v| ~ 7e12, where
    v^3 overflows and the reference's formula takes tanh(inf) = 1. Against the oracle's fp32 GELU: bit-identical."""
    M, N, K = 1024, 1032, 64
    rng = np.random.default_rng(12)
    xq = np.zeros((M, K), np.int8)
    xq[:, 0] = 1
    wq = np.zeros((N, K), np.int8)
    wq[:, 0] = 1
    sx = (np.where(np.arange(M) % 2, 1.0, -1.0) * 10.0 ** np.linspace(np.log10(20.0), 37.0, M)).astype(np.float32)
    sw = rng.uniform(0.5, 1.0, N).astype(np.float32)
    b = oracle.f2bf(rng.uniform(-0.05, 0.05, N).astype(np.float32))
    ref = oracle.gemm_i8_epilogue(np.ones((M, N), np.int32), sx, sw, b, True)
    assert not is_nan(ref).any()
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(dev(xq), dev(sx), dev(wq), dev(sw), dev_bf16(b), y, True)
    got = host_bits(y)
    assert not is_nan(got).any(), f"{int(is_nan(got).sum())} NaN outputs"
    u = ulp_dist(got, ref)
    assert int(u.max()) == 0, f"max {int(u.max())} ulp, {int((u > 0).sum())} outputs differ"
