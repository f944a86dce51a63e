"""Decode GEMVs on the GPU (through the C ABI via lfm2opt.kernels.ext()) against the CPU oracle.

Parity bar: bf16 outputs within max |err| / max |ref| <= 1e-2 (mean abs err reported); fused epilogues bit-identical
to the unfused ops of the same library, as the reference requires (tests/test_kernels.py:153-186). Shapes follow
tests/test_kernels.py:127-150 and the LFM2 decode step; batch sizes cover the B = 1 kernel, the MFMA kernel and the
chunking above 16 rows.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from conftest import GOLDEN
from gpu_util import assert_close_bf16, dev, dev_bf16, host_bits

pytestmark = pytest.mark.gpu

# the LFM2 decode step's GEMV shapes, plus the standalone 8192 x 2048 up-projection GEMV of the single-GEMV workload
DECODE_SHAPES = [(3072, 2048), (2048, 2048), (6144, 2048), (8192, 2048), (16384, 2048), (2048, 8192), (65536, 2048)]


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import ext

    return ext()


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


# ------------------------------------------------------------------------------------------------ fixtures
@pytest.mark.parametrize("name", ["gemv_w8_b1_n80_k1024", "gemv_w8_b3_n80_k1024", "gemv_w8_b16_n48_k2048",
                                  "gemv_w8_b20_n40_k512"])
def test_gemv_w8_fixture(E, name):
    f = load(name)
    B, N = f["y"].shape
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv(dev(f["W"]), dev(f["scale"]), dev_bf16(f["x"]), y)
    assert_close_bf16(host_bits(y), f["y"], what=name)


@pytest.mark.parametrize("name", ["gemv_bf16_b1_n48_k512", "gemv_bf16_b5_n48_k512"])
def test_gemv_bf16_fixture(E, name):
    f = load(name)
    B, N = f["y"].shape
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv(dev_bf16(f["W"]), None, dev_bf16(f["x"]), y)
    assert_close_bf16(host_bits(y), f["y"], what=name)


@pytest.mark.parametrize("name", ["swiglu_w8_b1_s40_k512", "swiglu_w8_b4_s48_k1024"])
def test_swiglu_fixture(E, name):
    f = load(name)
    B, S = f["y"].shape
    y = torch.empty(B, S, device="cuda", dtype=torch.bfloat16)
    E.gemv_epi(0, dev(f["W"]), dev(f["scale"]), dev_bf16(f["x"]), y)
    assert_close_bf16(host_bits(y), f["y"], what=name)


@pytest.mark.parametrize("name", ["residual_w8_b1_n64_k2048", "residual_w8_b16_n64_k1024"])
def test_residual_fixture(E, name):
    f = load(name)
    h = dev_bf16(f["h"])
    E.gemv_residual(dev(f["W"]), dev(f["scale"]), dev_bf16(f["x"]), h)
    assert_close_bf16(host_bits(h), f["h_out"], what=name)


def test_silu_mul_fixture(E):
    f = load("silu_mul_b3_i300")
    g = dev_bf16(f["g"])
    y = torch.empty(3, 300, device="cuda", dtype=torch.bfloat16)
    E.silu_mul(g, y)
    out = host_bits(y)
    assert_close_bf16(out, f["y"], what="silu_mul")
    from gpu_util import ulp_dist

    assert ulp_dist(out, f["y"]).max() <= 1  # exp differs from the host's by an ulp at most


# ------------------------------------------------------------------------------------------------ seeded parity
def _gen(seed, B, N, K):
    g = torch.Generator().manual_seed(seed)
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    scale = torch.randn(N, generator=g).abs() * 0.01 + 1e-3
    x = torch.randn(B, K, generator=g).to(torch.bfloat16)
    return W, scale, x


@pytest.mark.parametrize("B", [1, 2, 4, 8, 12, 16, 17, 24, 40, 64, 65])
@pytest.mark.parametrize("N,K", [(3072, 2048), (2048, 8192), (200, 1152), (96, 576), (40, 64)])
def test_gemv_w8_vs_oracle(E, B, N, K):
    W, scale, x = _gen(100 + B, B, N, K)
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv(W.cuda(), scale.cuda(), x.cuda(), y)
    ref = oracle.gemv(W.numpy(), scale.numpy(), x.view(torch.int16).numpy().view(np.uint16))
    assert_close_bf16(host_bits(y), ref, what=f"gemv int8 B={B} [{N}x{K}]")


MFMA_SHAPES = ["1,1,1", "1,1,4", "1,2,8", "1,2,1", "1,4,8", "1,4,1", "2,1,1", "2,1,2", "2,1,16",
               "2,1,1,2", "2,1,8,2", "1,1,1,2", "1,1,8,2", "1,2,2,2", "1,2,8,2", "1,4,1,2", "1,4,8,2", "1,1,1,4",
               "1,1,4,4", "1,2,2,4", "1,4,1,4", "1,4,4,4"]


def _launch_batches(shape):
    """Two batch sizes the forced shape accepts (KS = 2 takes 8 rows per batch tile, KS = 1 16)."""
    ks, bt = int(shape.split(",")[0]), int((shape.split(",") + ["1"])[3])
    if bt == 1:
        return (3, 8) if ks == 2 else (3, 13)
    top = (16 // ks) * bt
    return top // 2 + 3, top


@pytest.mark.parametrize("shape", MFMA_SHAPES)
@pytest.mark.parametrize("wt", ["int8", "bf16"])
def test_gemv_mfma_launch_shapes(E, tune, shape, wt):
    """Every matrix-core launch shape (k-parts KS, row tiles RT, wavefronts NWK, batch tiles BT, forced through
    LFM2Q_GEMV_MFMA) against the oracle, with a trailing half block (K = 1088), N not a multiple of the tile rows and
    a partial last batch tile; the residual epilogue bit-identical to the plain GEMV + add."""
    tune("LFM2Q_GEMV_MFMA", shape)
    N, K = 300, 1088
    g = torch.Generator().manual_seed(len(shape))
    for B in _launch_batches(shape):
        if wt == "int8":
            W, scale, x = _gen(B, B, N, K)
            ref = oracle.gemv(W.numpy(), scale.numpy(), host_bits(x))
            Wd, sd = W.cuda(), scale.cuda()
        else:
            W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
            x = torch.randn(B, K, generator=g).to(torch.bfloat16)
            ref = oracle.gemv(host_bits(W), None, host_bits(x))
            Wd, sd = W.cuda(), None
        y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
        E.gemv(Wd, sd, x.cuda(), y)
        assert_close_bf16(host_bits(y), ref, what=f"gemv {wt} shape {shape} B={B}")
        h0 = (torch.randn(B, N, generator=g) * 4).to(torch.bfloat16).cuda()
        h = h0.clone()
        E.gemv_residual(Wd, sd, x.cuda(), h)
        assert torch.equal(h, (h0.float() + y.float()).to(torch.bfloat16))


@pytest.mark.parametrize("rows", [1, 2, 4])
def test_gemv_w8_rows_hint_same_result(E, rows):
    """The rows-per-wavefront hint changes the launch shape only: per-row results are bit-identical."""
    W, scale, x = _gen(7, 1, 1000, 2048)
    W, scale, x = W.cuda(), scale.cuda(), x.cuda()
    y0 = torch.empty(1, 1000, device="cuda", dtype=torch.bfloat16)
    y1 = torch.empty_like(y0)
    E.gemv(W, scale, x, y0, 1)
    E.gemv(W, scale, x, y1, rows)
    assert torch.equal(y0, y1)


@pytest.mark.parametrize("wt,N,K", [("int8", 5000, 2048), ("int8", 3001, 8192), ("int8", 4000, 1024),
                                    ("bf16", 5000, 1024)])
def test_gemv_persistent_matches_one_shot(E, tune, wt, N, K):
    """Batch 1: the persistent kernel (forced with LFM2Q_GEMV_PERSIST=1; by default only for 131072+ rows at 8 wavefronts per CU) and the
    one-shot kernel give the same bits, plain, SwiGLU and residual, and match the oracle."""
    g = torch.Generator(device="cuda").manual_seed(N + K)
    if wt == "int8":
        W = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
        scale = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    else:
        W = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        scale = None
    x = torch.randn(1, K, device="cuda", generator=g).to(torch.bfloat16)
    h0 = (torch.randn(1, N, device="cuda", generator=g) * 4).to(torch.bfloat16)
    S = N // 2
    W2, s2 = W[:2 * S].contiguous(), None if scale is None else scale[:2 * S].contiguous()
    res = {}
    for mode in ("1", "0"):
        tune("LFM2Q_GEMV_PERSIST", mode)
        y = torch.empty(1, N, device="cuda", dtype=torch.bfloat16)
        E.gemv(W, scale, x, y)
        a = torch.empty(1, S, device="cuda", dtype=torch.bfloat16)
        E.gemv_epi(0, W2, s2, x, a)
        h = h0.clone()
        E.gemv_residual(W, scale, x, h)
        res[mode] = (y, a, h)
    for u, v in zip(res["1"], res["0"]):
        assert torch.equal(u, v)
    Wn = W.cpu().numpy() if wt == "int8" else host_bits(W)
    assert_close_bf16(host_bits(res["1"][0]), oracle.gemv(Wn, None if scale is None else scale.cpu().numpy(),
                                                          host_bits(x)), what=f"persistent gemv {wt} [{N}x{K}]")


@pytest.mark.parametrize("wt,N,K", [("int8", 2048, 8192), ("int8", 2050, 2048), ("int8", 3074, 2048),
                                    ("int8", 1030, 8192), ("int8", 102, 1024), ("int8", 38, 4096),
                                    ("bf16", 2054, 2048), ("bf16", 70, 512)])
@pytest.mark.parametrize("rows", ["1", "2", None])
def test_gemv_shared_activations_match_per_wavefront(E, tune, wt, N, K, rows):
    """Batch 1, one-shot kernel: the form whose workgroup stages the activation row in LDS (LFM2Q_GEMV_XS=1) gives
    the bits of the form where every wavefront loads it (=0), plain, SwiGLU and residual, at 1 / 2 / the automatic
    rows per wavefront. N not a multiple of the workgroup's rows: the last workgroup's wavefronts past the end take
    part in the shared load and store nothing."""
    g = torch.Generator(device="cuda").manual_seed(7 * N + K)
    if wt == "int8":
        W = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
        scale = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    else:
        W = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        scale = None
    x = torch.randn(1, K, device="cuda", generator=g).to(torch.bfloat16)
    h0 = (torch.randn(1, N, device="cuda", generator=g) * 4).to(torch.bfloat16)
    S = N // 2
    W2, s2 = W[:2 * S].contiguous(), None if scale is None else scale[:2 * S].contiguous()
    tune("LFM2Q_GEMV_PERSIST", 0)
    if rows:
        tune("LFM2Q_GEMV_R", rows)
    res = {}
    for mode in ("1", "0"):
        tune("LFM2Q_GEMV_XS", mode)
        y = torch.full((1, N), float("nan"), device="cuda", dtype=torch.bfloat16)
        E.gemv(W, scale, x, y)
        a = torch.full((1, S), float("nan"), device="cuda", dtype=torch.bfloat16)
        E.gemv_epi(0, W2, s2, x, a)
        h = h0.clone()
        E.gemv_residual(W, scale, x, h)
        res[mode] = (y, a, h)
    for u, v in zip(res["1"], res["0"]):
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))
    Wn = W.cpu().numpy() if wt == "int8" else host_bits(W)
    assert_close_bf16(host_bits(res["1"][0]), oracle.gemv(Wn, None if scale is None else scale.cpu().numpy(),
                                                          host_bits(x)), what=f"shared-x gemv {wt} [{N}x{K}]")


@pytest.mark.parametrize("N,K", DECODE_SHAPES)
@pytest.mark.parametrize("B", [1, 4, 16])
def test_gemv_w8_decode_shapes(E, N, K, B):
    """Full LFM2 decode shapes: against torch's fp32 dequant-matmul on the GPU (tests/test_kernels.py:137) and,
    on a sample of 64 rows, against the CPU oracle."""
    g = torch.Generator(device="cuda").manual_seed(N + K + B)
    W = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    scale = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    x = torch.randn(B, K, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv(W, scale, x, y)
    ref = F.linear(x.float(), W.float() * scale[:, None]).to(torch.bfloat16)
    assert_close_bf16(host_bits(y), host_bits(ref), what=f"gemv int8 B={B} [{N}x{K}] vs torch fp32")
    rows = torch.randperm(N, generator=torch.Generator().manual_seed(1))[:64].sort().values
    ro = oracle.gemv(W[rows.cuda()].cpu().numpy(), scale[rows.cuda()].cpu().numpy(), host_bits(x))
    assert_close_bf16(host_bits(y[:, rows.cuda()]), ro, what=f"gemv int8 B={B} [{N}x{K}] sampled rows vs oracle")


@pytest.mark.parametrize("B", [1, 3, 16, 20, 64])
@pytest.mark.parametrize("N,K", [(1040, 1024), (72, 576)])
def test_gemv_bf16_vs_oracle(E, B, N, K):
    g = torch.Generator().manual_seed(B)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(B, K, generator=g).to(torch.bfloat16)
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv(W.cuda(), None, x.cuda(), y)
    ref = oracle.gemv(W.view(torch.int16).numpy().view(np.uint16), None, x.view(torch.int16).numpy().view(np.uint16))
    assert_close_bf16(host_bits(y), ref, what=f"gemv bf16 B={B}")


@pytest.mark.parametrize("B", [2])
@pytest.mark.parametrize("wt,N,K", [("int8", 300, 2048), ("int8", 7000, 1024), ("bf16", 300, 1024),
                                    ("bf16", 6200, 512)])
def test_gemv_valu_batch_rows_match_batch_1(E, B, wt, N, K):
    """Batch 2 with short rows runs the VALU kernel over both batch rows at once: each row of the result equals a
    batch-1 call on that row bit for bit (plain, SwiGLU and residual), and the whole stays within the bar of the
    oracle."""
    g = torch.Generator(device="cuda").manual_seed(B * 100 + K)
    if wt == "int8":
        W = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
        scale = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    else:
        W = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        scale = None
    x = torch.randn(B, K, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv(W, scale, x, y)
    for b in range(B):
        y1 = torch.empty(1, N, device="cuda", dtype=torch.bfloat16)
        E.gemv(W, scale, x[b:b + 1].contiguous(), y1)
        assert torch.equal(y[b], y1[0]), f"row {b}"
    Wn = W.cpu().numpy() if wt == "int8" else host_bits(W)
    assert_close_bf16(host_bits(y), oracle.gemv(Wn, None if scale is None else scale.cpu().numpy(), host_bits(x)),
                      what=f"gemv {wt} B={B} [{N}x{K}] VALU batch")
    S = N // 2
    act = torch.empty(B, S, device="cuda", dtype=torch.bfloat16)
    E.gemv_epi(0, W[:2 * S].contiguous(), None if scale is None else scale[:2 * S].contiguous(), x, act)
    ref = torch.empty_like(act)
    E.silu_mul(y[:, :2 * S].contiguous(), ref)
    assert torch.equal(act, ref)
    h0 = (torch.randn(B, N, device="cuda", generator=g) * 4).to(torch.bfloat16)
    h = h0.clone()
    E.gemv_residual(W, scale, x, h)
    assert torch.equal(h, (h0.float() + y.float()).to(torch.bfloat16))


# ------------------------------------------------------------------------------------------------ fused epilogues
@pytest.mark.parametrize("B", [1, 2, 4, 8, 16, 19, 40, 64])
@pytest.mark.parametrize("wt", ["int8", "bf16"])
def test_swiglu_bit_identical_to_gemv_then_silu_mul(E, B, wt):
    """gemv_epi(0) == gemv + silu_mul bit for bit (tests/test_kernels.py:153-186), at the w1|w3 shape."""
    S, K = 8192, 2048
    g = torch.Generator(device="cuda").manual_seed(B)
    if wt == "int8":
        W = torch.randint(-127, 128, (2 * S, K), device="cuda", dtype=torch.int8, generator=g)
        scale = torch.rand(2 * S, device="cuda", generator=g) * 0.01 + 1e-3
    else:
        W = (torch.randn(2 * S, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        scale = None
    x = torch.randn(B, K, device="cuda", generator=g).to(torch.bfloat16)
    gg = torch.empty(B, 2 * S, device="cuda", dtype=torch.bfloat16)
    E.gemv(W, scale, x, gg)
    ref = torch.empty(B, S, device="cuda", dtype=torch.bfloat16)
    E.silu_mul(gg, ref)
    out = torch.empty_like(ref)
    E.gemv_epi(0, W, scale, x, out)
    assert torch.equal(out, ref), (out.float() - ref.float()).abs().max()


@pytest.mark.parametrize("B", [1, 4, 8, 12, 16, 24, 64])
def test_residual_bit_identical_to_gemv_then_add(E, B):
    N, K = 2048, 8192
    g = torch.Generator(device="cuda").manual_seed(B)
    W = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    scale = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    x = torch.randn(B, K, device="cuda", generator=g).to(torch.bfloat16)
    h = (torch.randn(B, N, device="cuda", generator=g) * 4).to(torch.bfloat16)
    y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
    E.gemv(W, scale, x, y)
    ref = (h.float() + y.float()).to(torch.bfloat16)
    E.gemv_residual(W, scale, x, h)
    assert torch.equal(h, ref)


# ------------------------------------------------------------------------------------------------ argument errors
def test_argument_errors_raise_before_launch(E):
    W = torch.zeros(64, 512, device="cuda", dtype=torch.int8)
    s = torch.ones(64, device="cuda")
    x = torch.zeros(1, 512, device="cuda", dtype=torch.bfloat16)
    y = torch.zeros(1, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="int8 W needs fp32 scale"):
        E.gemv(W, None, x, y)
    with pytest.raises(RuntimeError, match=r"x \[B, K\], y \[B, N\]"):
        E.gemv(W, s, x, torch.zeros(1, 63, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="multiple of 64"):
        E.gemv(torch.zeros(64, 96, device="cuda", dtype=torch.int8), s, torch.zeros(1, 96, device="cuda",
               dtype=torch.bfloat16), y)
    with pytest.raises(RuntimeError, match="must be contiguous CUDA bf16"):
        E.gemv(W, s, x.float(), y)
    with pytest.raises(RuntimeError, match="short-conv"):
        E.gemv_epi(1, W, s, x, y)
    torch.cuda.synchronize()


def test_single_gemv_8192x2048_full_oracle(E):
    """The standalone decode up-projection: x bf16 [1, 2048] ~ N(0, 1), W int8 [8192, 2048] uniform over [-127, 127],
    scale |N(0, 1)| 0.01 + 1e-3, y = bf16((x W^T) scale), seeded. Every output against the CPU oracle and against
    the reference's PyTorch dequant-matmul (tests/test_kernels.py:137) evaluated on the CPU in fp32."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 2048, generator=g).to(torch.bfloat16)
    W = torch.randint(-127, 128, (8192, 2048), generator=g, dtype=torch.int8)
    scale = torch.randn(8192, generator=g).abs() * 0.01 + 1e-3
    y = torch.empty(1, 8192, device="cuda", dtype=torch.bfloat16)
    E.gemv(W.cuda(), scale.cuda(), x.cuda(), y)
    out = host_bits(y)
    assert_close_bf16(out, oracle.gemv(W.numpy(), scale.numpy(), host_bits(x)), what="gemv 8192x2048 vs oracle")
    ref = F.linear(x.float(), W.float() * scale[:, None]).to(torch.bfloat16)
    assert_close_bf16(out, host_bits(ref), what="gemv 8192x2048 vs CPU dequant-matmul")
