"""The per-token W8A8 layer behind one call (lfm2q_gemm_i8_fq, through lfm2opt.kernels.int8_ext().gemm_i8_fq), on
its one-launch kernel (tuning knob LFM2Q_GEMM_FQ = 1, set for every test here but the last): the persistent GEMM's
workgroups quantize the bf16 activations themselves before their tiles.

Parity bar: bit-identical to the pair it replaces -- quant_rows, then gemm_i8 with the same workspace -- in all three
outputs (the int8 rows, the scales, y) on the LFM2 prefill and SigLIP2 shapes, ragged M / N / K, every persistent
tile form and K split, with bias and GELU; the shapes the persistent kernel does not take run the pair itself. The
steal path (a waiting workgroup quantizing chunks that are still open, forced by a zero wait bound), back-to-back
calls of different sizes on one workspace (the control block's epochs), calls interleaved with K-split GEMMs on the
same workspace and graph replays are bit-identical too. One small case is checked against the oracle directly."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import host_bits, ulp_dist

pytestmark = pytest.mark.gpu

PREFILL = [(M, K, N) for M in (512, 2048, 4096) for K, N in ((2048, 3072), (2048, 16384), (8192, 2048))]
VISION = [(10240, 1152, 3456), (10240, 1152, 1152), (10240, 1152, 4304), (10240, 4304, 1152)]


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import int8_ext

    return int8_ext()


@pytest.fixture(autouse=True)
def one_launch(request, tune):
    if "default_dispatch" not in request.node.name:
        tune("LFM2Q_GEMM_FQ", 1)


def activations(seed, M, K):
    """~N(0, 1) with 0.1 % outliers at 20 sigma (the prefill workload)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    out = torch.rand(M, K, generator=g) < 1e-3
    x[out] = 20.0 * torch.sign(torch.randn(int(out.sum()), generator=g))
    return x.to(torch.bfloat16).cuda()


def weights(seed, N, K, bias):
    g = torch.Generator().manual_seed(seed + 1)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    sw = (torch.rand(N, generator=g) * 1e-3 + 1e-4).cuda()
    b = torch.randn(N, generator=g).to(torch.bfloat16).cuda() if bias else None
    return w, sw, b


def pair(E, x, w, sw, b, gelu):
    M, K = x.shape
    q = torch.empty(M, K, device="cuda", dtype=torch.int8)
    s = torch.empty(M, device="cuda")
    E.quant_rows(x, q, s)
    y = torch.empty(M, w.shape[0], device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(q, s, w, sw, b, y, gelu)
    return q, s, y


def fused(E, x, w, sw, b, gelu):
    M, K = x.shape
    q = torch.full((M, K), 99, device="cuda", dtype=torch.int8)
    s = torch.full((M,), -1.0, device="cuda")
    y = torch.full((M, w.shape[0]), 7.0, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8_fq(x, q, s, w, sw, b, y, gelu)
    return q, s, y


def assert_same(got, ref, what):
    for name, a, r in zip(("q", "sx", "y"), got, ref):
        diff = int((a.view(torch.uint8) != r.view(torch.uint8)).sum())
        assert diff == 0, f"{what}: {diff} bytes of {name} differ from quant_rows + gemm_i8"


@pytest.mark.parametrize("M,K,N", PREFILL + VISION)
def test_fq_equals_pair_full_shapes(E, M, K, N):
    """The 13 W8A8 prefill / vision shapes, bias and GELU on the vision fc1 form (N = 4304)."""
    x = activations(M + K + N, M, K)
    w, sw, b = weights(N, N, K, N in (4304, 3456))
    gelu = N == 4304
    assert_same(fused(E, x, w, sw, b, gelu), pair(E, x, w, sw, b, gelu), f"{M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N,bias,gelu", [(1, 16, 8, False, False), (37, 1152, 200, True, True),
                                             (777, 4304, 1160, True, False), (3, 16384, 512, False, True),
                                             (1000, 16, 64, True, False), (17, 2048, 3072, False, False),
                                             (255, 96, 4104, True, True), (5, 16400, 256, False, False),
                                             (9, 2048, 100, True, False)])
def test_fq_equals_pair_ragged(E, M, K, N, bias, gelu):
    """Ragged M / N / K: one row, K = 16 (1024-row chunks), K = 16384 (one row per chunk), chunks cut by M; the last
    two run the pair inside the call (K > 16384; N % 8 != 0)."""
    x = activations(M * 3 + K, M, K)
    w, sw, b = weights(N + K, N, K, bias)
    assert_same(fused(E, x, w, sw, b, gelu), pair(E, x, w, sw, b, gelu), f"{M}x{K}x{N}")


@pytest.mark.parametrize("bm,bn,sk", [(256, 256, 1), (256, 128, 1), (128, 128, 1), (128, 64, 1), (256, 128, 2),
                                      (128, 128, 3), (128, 64, 4)])
@pytest.mark.parametrize("M,K,N", [(64, 8192, 2048), (600, 2048, 1032)])
def test_fq_every_tile_form(E, tune, bm, bn, sk, M, K, N):
    """Each persistent tile form, unsplit and with K cut over workgroups, forced through the tile knobs."""
    x = activations(bm + bn + sk + M, M, K)
    w, sw, b = weights(M + N, N, K, True)
    ref = pair(E, x, w, sw, b, False)
    tune("LFM2Q_GEMM_BM", bm)
    tune("LFM2Q_GEMM_BN", bn)
    tune("LFM2Q_GEMM_SPLITK", sk)
    assert_same(fused(E, x, w, sw, b, False), ref, f"{bm}x{bn}/{sk} {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(512, 8192, 2048), (2048, 2048, 3072), (10240, 1152, 1152), (1, 16, 8)])
def test_fq_steal_path(E, tune, M, K, N):
    """A zero wait bound: every workgroup that finds a chunk still open at its first poll quantizes (and publishes)
    every open chunk itself, so chunks are written several times over; the outputs stay bit-identical."""
    x = activations(K + 5, M, K)
    w, sw, b = weights(N, N, K, True)
    ref = pair(E, x, w, sw, b, True)
    tune("LFM2Q_GEMM_FQ_WAIT_US", 0)
    for _ in range(3):
        assert_same(fused(E, x, w, sw, b, True), ref, f"steal {M}x{K}x{N}")


def test_fq_back_to_back_and_with_split_calls(E, tune):
    """Calls of different sizes in a row on one workspace (each launch advances the control block's epoch, so the
    earlier calls' done states mean nothing to the next), a smaller M after a larger one (stale q rows and states
    past the new M), and K-split gemm_i8 calls on the same workspace between them."""
    cases = [(2048, 2048, 3072), (512, 8192, 2048), (37, 1152, 200), (4096, 2048, 16384), (512, 8192, 2048),
             (1, 16, 8), (600, 2048, 1032)]
    for i, (M, K, N) in enumerate(cases):
        x = activations(100 + i, M, K)
        w, sw, b = weights(200 + i, N, K, i % 2 == 0)
        got = fused(E, x, w, sw, b, i % 3 == 0)
        ref = pair(E, x, w, sw, b, i % 3 == 0)
        assert_same(got, ref, f"call {i}: {M}x{K}x{N}")
        tune("LFM2Q_GEMM_SPLITK", 4)  # a K-split GEMM on the same workspace between two fused calls
        xs = activations(300 + i, 64, 8192)
        ws_, sws, _ = weights(400 + i, 2048, 8192, False)
        pair(E, xs, ws_, sws, None, False)
        tune("LFM2Q_GEMM_SPLITK", 0)


def test_fq_against_the_oracle(E):
    """A small case straight against the oracle: quant_rows (q, s bit-exact) and the GEMM epilogue (0 bf16 ulp)."""
    M, K, N = 40, 1152, 136
    x = activations(11, M, K)
    w, sw, b = weights(12, N, K, True)
    q, s, y = fused(E, x, w, sw, b, False)
    rq, rs = oracle.quant_rows(host_bits(x))
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.cpu().numpy(), rq)
    acc = oracle.gemm_i8_i32(rq, w.cpu().numpy())
    ref = oracle.gemm_i8_epilogue(acc, rs, sw.cpu().numpy(), host_bits(b), False)
    assert int(ulp_dist(host_bits(y), ref).max()) == 0


def test_fq_graph_replays(E):
    """Captured once, replayed with new activations copied into the input between replays (eager work and
    synchronizations in between): every replay equals the eager pair on that input."""
    from lfm2opt import _capi

    M, K, N = 512, 8192, 2048
    w, sw, b = weights(7, N, K, True)
    x = activations(1, M, K)
    q = torch.empty(M, K, device="cuda", dtype=torch.int8)
    s = torch.empty(M, device="cuda")
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    cap = torch.cuda.Stream()
    _capi.prepare_workspace(x.device, cap)
    E.gemm_i8_fq(x, q, s, w, sw, b, y, False)  # warm up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        E.gemm_i8_fq(x, q, s, w, sw, b, y, False)
    for i in range(4):
        xi = activations(50 + i, M, K)
        x.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        assert_same((q, s, y), pair(E, xi, w, sw, b, False), f"replay {i}")


def test_fq_argument_errors(E):
    from lfm2opt import _capi

    x = torch.zeros(4, 64, device="cuda", dtype=torch.bfloat16)
    q = torch.zeros(4, 64, device="cuda", dtype=torch.int8)
    s = torch.zeros(4, device="cuda")
    w = torch.zeros(8, 64, device="cuda", dtype=torch.int8)
    sw = torch.ones(8, device="cuda")
    y = torch.zeros(4, 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="xq shape"):
        E.gemm_i8_fq(x, q[:2], s, w, sw, None, y, False)
    with pytest.raises(RuntimeError, match="sx shape"):
        E.gemm_i8_fq(x, q, s[:3], w, sw, None, y, False)
    small = torch.zeros(1 << 20, device="cuda", dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="workspace"):
        _capi.call("lfm2q_gemm_i8_fq", x.data_ptr(), q.data_ptr(), s.data_ptr(), w.data_ptr(), sw.data_ptr(), None,
                   y.data_ptr(), 4, 8, 64, 0, small.data_ptr(), small.numel(), _capi.stream(x))
    with pytest.raises(RuntimeError, match="null pointer"):
        _capi.call("lfm2q_gemm_i8_fq", x.data_ptr(), q.data_ptr(), s.data_ptr(), w.data_ptr(), sw.data_ptr(), None,
                   y.data_ptr(), 4, 8, 64, 0, None, 0, _capi.stream(x))
    torch.cuda.synchronize()


@pytest.mark.parametrize("M,K,N", [(512, 2048, 3072), (37, 1152, 200)])
def test_fq_default_dispatch_is_the_pair(E, M, K, N):
    """Without the knob the call runs quant_rows and gemm_i8: the same three outputs."""
    x = activations(M + 1, M, K)
    w, sw, b = weights(N + 1, N, K, True)
    assert_same(fused(E, x, w, sw, b, True), pair(E, x, w, sw, b, True), f"default {M}x{K}x{N}")
