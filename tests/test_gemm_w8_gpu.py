"""W8A16 GEMM (bf16 activations x int8 weights, fp32 accumulation on the bf16 matrix cores) on the GPU.

Parity bar: the reference's own rule (tests/test_int8_gemm.py:178-195): relative Frobenius error against the fp64
result at most 1.5 x that of the platform BLAS on the dequantized bf16 weights, + 1e-4; and per element
max |err| / max |ref| <= 1e-2 against the CPU oracle (fp64 accumulation rounded once), on small shapes in full and
on sampled rows of the full shapes.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from gpu_util import assert_close_bf16, dev, dev_bf16, host_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import int8_ext

    return int8_ext()


def operands(seed, M, K, N, bias):
    r = np.random.default_rng(seed)
    x = oracle.f2bf(r.standard_normal((M, K)).astype(np.float32))
    W = r.integers(-127, 128, (N, K), dtype=np.int8)
    sw = (np.abs(r.standard_normal(N)) * 0.01 + 1e-3).astype(np.float32)
    b = oracle.f2bf(r.standard_normal(N).astype(np.float32)) if bias else None
    return x, W, sw, b


def run(E, x, W, sw, b, gelu):
    y = torch.empty(x.shape[0], W.shape[0], device="cuda", dtype=torch.bfloat16)
    E.gemm_w8(dev_bf16(x), dev(W), dev(sw), None if b is None else dev_bf16(b), y, gelu)
    return host_bits(y)


@pytest.mark.parametrize("M,K,N,bias,gelu", [(37, 320, 24, True, False), (70, 1152, 100, False, False),
                                             (33, 576, 40, True, True), (129, 4304, 72, True, False),
                                             (1, 2048, 264, False, False)])
def test_gemm_w8_vs_oracle(E, M, K, N, bias, gelu):
    x, W, sw, b = operands(M + K + N, M, K, N, bias)
    assert_close_bf16(run(E, x, W, sw, b, gelu), oracle.gemm_w8(x, W, sw, b, gelu),
                      what=f"gemm_w8 {M}x{K}x{N}{' bias' if bias else ''}{' gelu' if gelu else ''}")


@pytest.mark.parametrize("tile,ksplit", [(t, k) for t in ("128x128", "128x64", "64x128", "64x64") for k in (1, 2)]
                         + [("64x64", 4)])
def test_gemm_w8_every_tile(E, tile, ksplit, tune):
    """Every tile with K split over 1, 2 or 4 wavefront groups (LFM2Q_GEMM_KSPLIT), with K = 576 (9 stages), 1104
    (18 stages, uneven split) and 128 (2 stages: some groups have nothing to add)."""
    bm, bn = tile.split("x")
    tune("LFM2Q_GEMM_BM", bm)
    tune("LFM2Q_GEMM_BN", bn)
    tune("LFM2Q_GEMM_KSPLIT", str(ksplit))
    for K in (576, 1104, 128):
        x, W, sw, b = operands(3 + K, 200, K, 264, True)
        assert_close_bf16(run(E, x, W, sw, b, False), oracle.gemm_w8(x, W, sw, b),
                          what=f"gemm_w8 tile {tile} ksplit {ksplit} K={K}")


@pytest.mark.parametrize("M,K,N,bias,gelu", [(64, 2048, 16384, False, False), (256, 8192, 2048, False, False),
                                             (10240, 1152, 4304, True, True)])
def test_gemm_w8_full_shape_error_rule(E, M, K, N, bias, gelu):
    g = torch.Generator(device="cuda").manual_seed(M + N)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
    from lfm2opt.quant import quantize_int8

    wq, sw = quantize_int8(w)
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_w8(x, wq, sw, b, y, gelu)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(0))[:64].sort().values.cuda()
    r64 = (x[rows].double() @ wq.double().t()) * sw.double()[None, :]
    if b is not None:
        r64 = r64 + b.double()
    wd = (wq.float() * sw[:, None]).to(torch.bfloat16)
    rc = F.linear(x[rows].float(), wd.float(), None if b is None else b.float()).to(torch.bfloat16)
    if gelu:
        r64 = F.gelu(r64, approximate="tanh")
        rc = F.gelu(rc.float(), approximate="tanh").to(torch.bfloat16)
    e_ours = ((y[rows].double() - r64).norm() / r64.norm()).item()
    e_blas = ((rc.double() - r64).norm() / r64.norm()).item()
    print(f"gemm_w8 {M}x{K}x{N}: rel err {e_ours:.3e} (torch on dequantized bf16 W {e_blas:.3e})")
    assert e_ours <= 1.5 * e_blas + 1e-4
    ro = oracle.gemm_w8(host_bits(x[rows]), wq.cpu().numpy(), sw.cpu().numpy(),
                        None if b is None else host_bits(b), gelu)
    assert_close_bf16(host_bits(y[rows]), ro, what=f"gemm_w8 {M}x{K}x{N} sampled rows vs oracle")


def test_int8_linear_w8a16(cuda):
    from lfm2opt.int8 import Int8Linear
    from lfm2opt.kernels import int8_ext

    g = torch.Generator(device="cuda").manual_seed(6)
    w = (torch.randn(192, 1152, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(192, device="cuda", generator=g).to(torch.bfloat16)
    x = torch.randn(4, 7, 1152, device="cuda", generator=g).to(torch.bfloat16)
    lin = Int8Linear(w, b, a8=False)
    y = lin(x, gelu=True)
    ref = torch.empty(28, 192, device="cuda", dtype=torch.bfloat16)
    int8_ext().gemm_w8(x.reshape(28, 1152), lin.q, lin.s, b, ref, True)
    assert torch.equal(y.reshape(28, 192), ref)


@pytest.mark.parametrize("tile", ["128x128", "64x64"])
@pytest.mark.parametrize("sk", [2, 3, 8])
def test_gemm_w8_split_k_across_workgroups(E, tile, sk, tune):
    """K cut into SK slices over workgroups (LFM2Q_GEMM_SPLITK), the fp32 partial tiles summed in slice order through
    the stream's workspace by the last workgroup of each tile: against the oracle as every W8A16 call, on ragged
    shapes with K of 69 stages (unequal slices) and 9 stages (some slices empty at SK = 8); two calls in a row give
    the same bits (the sum order does not depend on which workgroup finishes last, and the counters are back at 0)."""
    bm, bn = tile.split("x")
    tune("LFM2Q_GEMM_BM", bm)
    tune("LFM2Q_GEMM_BN", bn)
    tune("LFM2Q_GEMM_SPLITK", str(sk))
    for M, K, N, bias, gelu in [(70, 4416, 136, True, False), (33, 576, 264, False, True)]:
        x, W, sw, b = operands(M + K + N + sk, M, K, N, bias)
        y1 = run(E, x, W, sw, b, gelu)
        y2 = run(E, x, W, sw, b, gelu)
        assert np.array_equal(y1, y2), "two split calls differ"
        assert_close_bf16(y1, oracle.gemm_w8(x, W, sw, b, gelu), what=f"gemm_w8 split {sk} {tile} {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(256, 8192, 2048), (64, 8192, 2048)])
def test_gemm_w8_split_k_automatic(E, M, K, N):
    """The decode-batch shapes whose tiles leave most CUs idle (w2: N = 2048, K = 8192), where the automatic choice
    cuts K over workgroups: 64 sampled rows against the oracle; repeated calls bit-identical."""
    x, W, sw, b = operands(M + K + N, M, K, N, False)
    y1 = run(E, x, W, sw, b, False)
    assert np.array_equal(y1, run(E, x, W, sw, b, False))
    rows = np.sort(np.random.default_rng(3).permutation(M)[:64])
    assert_close_bf16(y1[rows], oracle.gemm_w8(x[rows], W, sw, b, False), what=f"gemm_w8 auto split {M}x{K}x{N}")
