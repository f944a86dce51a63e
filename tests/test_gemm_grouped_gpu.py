"""Grouped-64 W8A8 GEMM and its INT8-output form on the GPU (through the C ABI via lfm2opt.kernels.int8_ext()).

Parity bar: the grouped fold is the reference's operation sequence (exact int32 partial per 64-wide K group,
facc = fma((float)part, sxT[g, m], facc) in group order, then facc * sw + b), so the bf16 output is bit-exact against
the oracle without GELU and within 1 bf16 ulp with it, or one fp32 ulp of the GELU input in absolute value where the
formula's 1 + tanh cancels for inputs well below 0 (tests/test_int8_gemm.py:81-104 accepts far more: 1.05 x the
bf16 rounding error of the exact result, also checked here at full shape); gemm_i8_q is bit-identical to the grouped
gemm_i8 followed by grouped quant_rows (tests/test_int8_gemm.py:107-120).
"""

import os

import numpy as np
import pytest
import torch

import oracle
import rounding_cases
from gpu_util import dev, dev_bf16, host_bits, ulp_dist

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import int8_ext

    return int8_ext()


def operands(seed, M, K, N, bias):
    r = np.random.default_rng(seed)
    x = oracle.f2bf(r.standard_normal((M, K)).astype(np.float32))
    x[:, 7] = oracle.f2bf(np.full(M, 25.0, np.float32))  # an outlier channel: its group gets a large scale
    w = oracle.f2bf((r.standard_normal((N, K)) * 0.02).astype(np.float32))
    xq, sxT = oracle.quant_groups(x)
    wq, sw = oracle.quant_rows(w)
    b = oracle.f2bf(r.standard_normal(N).astype(np.float32)) if bias else None
    return xq, sxT, wq, sw, b


def run_grouped(E, xq, sxT, wq, sw, b, gelu):
    M, N = xq.shape[0], wq.shape[0]
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(dev(xq), dev(sxT), dev(wq), dev(sw), None if b is None else dev_bf16(b), y, gelu)
    return y


@pytest.mark.parametrize("M,K,N,bias,gelu", [(37, 320, 24, True, False), (300, 1152, 520, False, False),
                                             (129, 4352, 72, True, False), (65, 2048, 3072, False, True),
                                             (17, 256, 1000, True, True)])
def test_gemm_grouped_vs_oracle(E, M, K, N, bias, gelu):
    xq, sxT, wq, sw, b = operands(M + K + N, M, K, N, bias)
    y = run_grouped(E, xq, sxT, wq, sw, b, gelu)
    ref = oracle.gemm_i8_grouped(xq, sxT, wq, sw, b, gelu)
    u = int(ulp_dist(host_bits(y), ref).max())
    assert u <= (1 if gelu else 0), f"{u} bf16 ulp"


def force_form(tune, stages):
    """stages: "default" (the automatic form), "3" (the 3-stage ring, pipelined fold), "pipe" / "seq" (the 128 x 128
    kernel's pipelined / tile-sequential fold, LFM2Q_GEMM_GSEQ = 0 / 1)."""
    if stages == "3":
        tune("LFM2Q_GEMM_STAGES", "3")
    elif stages in ("pipe", "seq"):
        tune("LFM2Q_GEMM_GSEQ", "1" if stages == "seq" else "0")


@pytest.mark.parametrize("tile,stages", [(t, st) for t in ("128x128", "128x64", "64x128", "64x64")
                                         for st in ("default", "3")] + [("128x128", "seq")])
def test_gemm_grouped_every_tile(E, tile, stages, tune):
    """Each tile on the default 4-stage LDS ring and on the 3-stage one (LFM2Q_GEMM_STAGES = 3), and the 128 x 128
    kernel's tile-sequential fold (LFM2Q_GEMM_GSEQ = 1)."""
    bm, bn = tile.split("x")
    tune("LFM2Q_GEMM_BM", bm)
    tune("LFM2Q_GEMM_BN", bn)
    force_form(tune, stages)
    xq, sxT, wq, sw, b = operands(5, 200, 576, 264, True)
    y = run_grouped(E, xq, sxT, wq, sw, b, False)
    assert np.array_equal(host_bits(y), oracle.gemm_i8_grouped(xq, sxT, wq, sw, b))


@pytest.mark.parametrize("tile", [None, "128x128", "128x64", "64x128", "64x64"])
def test_gemm_grouped_rounding_points(E, tile, tune):
    """Operands whose bf16 outputs depend on each rounding point of the fold and the epilogue (tests/rounding_cases.py,
    expected bits derived by hand: an fma per group in group order into an fp32 accumulator, then fl(fl(facc sw) +
    b)), on every grouped tile, the pipelined fold of the tiles with several 32 x 32 blocks per wavefront included."""
    if tile:
        bm, bn = tile.split("x")
        tune("LFM2Q_GEMM_BM", bm)
        tune("LFM2Q_GEMM_BN", bn)
    xq, sxT, wq, sw, b, expect = rounding_cases.grouped_fold_case()
    y = host_bits(run_grouped(E, xq, sxT, wq, sw, b, False))
    for (m, n), bits in expect.items():
        assert int(y[m, n]) == bits, (m, n, hex(int(y[m, n])))
    assert np.array_equal(y, oracle.gemm_i8_grouped(xq, sxT, wq, sw, b))


@pytest.mark.parametrize("stages", ["default", "3", "seq"])
@pytest.mark.parametrize("K", [64, 128, 192, 448, 704])
def test_gemm_grouped_ring_rounds(E, K, stages, tune):
    """K of 1-3 groups (fewer stages than the ring has slots) and of 7 and 11 groups (every partial last round of
    both ring depths; "seq": the 128 x 128 tile-sequential fold, whose first fold is the stage -1 one and whose last
    tile is folded after the loop), bit-exact against the oracle."""
    if stages == "seq":
        tune("LFM2Q_GEMM_BM", "128")
        tune("LFM2Q_GEMM_BN", "128")
    force_form(tune, stages)
    xq, sxT, wq, sw, b = operands(K + 3, 150, K, 200, True)
    y = run_grouped(E, xq, sxT, wq, sw, b, False)
    assert np.array_equal(host_bits(y), oracle.gemm_i8_grouped(xq, sxT, wq, sw, b))


GROUPED_FULL = ([(M, K, N, False, False) for M in (512, 2048, 4096) for K, N in ((2048, 3072), (2048, 16384),
                                                                                  (8192, 2048))]
                + [(10240, 1152, 3456, True, False), (10240, 1152, 1152, True, False), (10240, 1152, 4304, True, True)])


@pytest.mark.parametrize("M,K,N,bias,gelu", GROUPED_FULL)
def test_gemm_grouped_every_configuration_full_shapes(E, M, K, N, bias, gelu, tune):
    """Every grouped tile on both ring depths (and the 128 x 128 kernel's pipelined and tile-sequential folds, each
    forced) at the full prefill / vision shapes whose K is a multiple of 64, on
    grouped-quantized ~N(0,1) activations with 0.1 % outliers at 20 sigma, two calls each: bit-identical to the
    automatic choice, whose sampled rows equal the oracle's fold (<= 1 ulp with GELU)."""
    g = torch.Generator(device="cuda").manual_seed(M + K + N + 5)
    wq = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
    x = torch.randn(M, K, device="cuda", generator=g)
    x[torch.rand(M, K, device="cuda", generator=g) < 1e-3] = 20.0
    xq = torch.empty(M, K, device="cuda", dtype=torch.int8)
    sxT = torch.empty(K // 64, M, device="cuda")
    E.quant_rows(x.to(torch.bfloat16), xq, sxT)
    base = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(xq, sxT, wq, sw, b, base, gelu)
    rows = np.array([0, M // 3, M - 1])
    args = (xq[rows].cpu().numpy(), sxT[:, rows].cpu().numpy(), wq.cpu().numpy(), sw.cpu().numpy(),
            None if b is None else host_bits(b))
    o = oracle.gemm_i8_grouped(*args, gelu)
    u = ulp_dist(host_bits(base[rows]), o)
    if gelu:
        # where 1 + tanh(.) cancels in fp32 (v well below 0, the reference's formula) the result is tiny and a one-ulp
        # difference in tanh becomes several bf16 ulps of it: there the bar is one fp32 ulp of v in absolute value
        v = oracle.bf2f(oracle.gemm_i8_grouped(*args, False)).astype(np.float64)
        d = np.abs(oracle.bf2f(host_bits(base[rows])).astype(np.float64) - oracle.bf2f(o).astype(np.float64))
        ok = (u <= 1) | ((v < 0) & (d <= 2.0 ** -22 * np.abs(v)))
        assert ok.all(), f"{int((~ok).sum())} outputs off, max {int(u.max())} ulp"
    else:
        assert int(u.max()) == 0
    y = torch.empty_like(base)
    for tile in ("128x128", "128x64", "64x128", "64x64"):
        bm, bn = tile.split("x")
        tune("LFM2Q_GEMM_BM", bm)
        tune("LFM2Q_GEMM_BN", bn)
        for stages in ("default", "3") + (("pipe", "seq") if tile == "128x128" else ()):
            tune("LFM2Q_GEMM_STAGES", None)
            tune("LFM2Q_GEMM_GSEQ", None)
            force_form(tune, stages)
            for call in range(2):
                y.fill_(3.0)
                E.gemm_i8(xq, sxT, wq, sw, b, y, gelu)
                assert torch.equal(y.view(torch.int16), base.view(torch.int16)), (tile, stages, call)


@pytest.mark.parametrize("stages", ["4", "3"])
def test_gemm_grouped_64x64_full_occupancy(E, stages, tune):
    """The 64 x 64 grouped kernel (one 32 x 32 block per wavefront, whose fold the compiler sinks below the next
    stage's barrier) at 4096 x 2048 x 16384: 16384 workgroups, 4-5 resident per CU, LDS busy. Before its stage
    barrier waited for the LDS reads, a stage's scale read could be overtaken by the refill of its slot (seen once, at
    the 3-stage ring); every call must equal the 128 x 128 kernel bit for bit, and sampled rows the oracle."""
    M, K, N = 4096, 2048, 16384
    g = torch.Generator(device="cuda").manual_seed(41)
    wq = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    xq = torch.empty(M, K, device="cuda", dtype=torch.int8)
    sxT = torch.empty(K // 64, M, device="cuda")
    E.quant_rows(x, xq, sxT)
    tune("LFM2Q_GEMM_BM", "128")
    tune("LFM2Q_GEMM_BN", "128")
    ref = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(xq, sxT, wq, sw, None, ref, False)
    tune("LFM2Q_GEMM_BM", "64")
    tune("LFM2Q_GEMM_BN", "64")
    tune("LFM2Q_GEMM_STAGES", stages)
    y = torch.empty_like(ref)
    for call in range(4):
        y.fill_(3.0)
        E.gemm_i8(xq, sxT, wq, sw, None, y, False)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"call {call}"
    rows = np.array([0, 1, 63, 64, 2047, 4095])
    o = oracle.gemm_i8_grouped(xq[rows].cpu().numpy(), sxT[:, rows].cpu().numpy(), wq.cpu().numpy(),
                               sw.cpu().numpy())
    assert np.array_equal(host_bits(y[rows]), o)


@pytest.mark.skip(reason="a persistent grouped-64 kernel (two groups per 128-byte stage, scale ring in LDS) faulted "
                         "the GPU on this case, its first run with more tiles than workgroups (128 x 64 tiles, "
                         "1100 x 320 x 2056). Cause since found on the CPU: an inline-asm direct-to-LDS load read a "
                         "buffer resource that v_readlane_b32 had restored with no wait states (a stale base); "
                         "every such load now has the wait states and the build checks for the hazard, but the "
                         "kernel stays out of the library, so the grouped path runs the one-tile-per-workgroup "
                         "kernels and this case stays off the GPU")
@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64"])
@pytest.mark.parametrize("gelu", [False, True])
def test_gemm_grouped_persistent_many_tiles(E, tile, gelu, tune):
    """The persistent grouped kernels with more tiles than workgroups (one workgroup per CU takes several tiles, the
    next tile's first stages and scale slots loading during the previous tile's epilogue), M / N tails and K of 5
    groups: bit-exact against the oracle's fold (<= 1 ulp with GELU) and bit-identical to the one-tile-per-workgroup
    grouped kernel of the same tile where there is one."""
    bm, bn = tile.split("x")
    tune("LFM2Q_GEMM_BM", bm)
    tune("LFM2Q_GEMM_BN", bn)
    M, K, N = 1100, 320, 2056
    xq, sxT, wq, sw, b = operands(11 + int(gelu), M, K, N, True)
    y = host_bits(run_grouped(E, xq, sxT, wq, sw, b, gelu))
    ref = oracle.gemm_i8_grouped(xq, sxT, wq, sw, b, gelu)
    assert int(ulp_dist(y, ref).max()) <= (1 if gelu else 0)
    if bm == "128":
        tune("LFM2Q_GEMM_BIGP", "0")
        assert np.array_equal(y, host_bits(run_grouped(E, xq, sxT, wq, sw, b, gelu)))


@pytest.mark.parametrize("M,K,N", [(2048, 2048, 16384), (4096, 8192, 2048)])
def test_gemm_grouped_full_shape_error_rule(E, M, K, N):
    """Full LFM2 prefill shapes: against the exact fp64 per-group sum on the GPU, the reference's rule (relative
    Frobenius error <= 1.05 x that of the bf16 rounding of the exact result), and 48 sampled rows against the
    oracle bit for bit."""
    g = torch.Generator(device="cuda").manual_seed(M + N)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    wq = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    xq = torch.empty(M, K, device="cuda", dtype=torch.int8)
    sxT = torch.empty(K // 64, M, device="cuda")
    E.quant_rows(x, xq, sxT)
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(xq, sxT, wq, sw, None, y, False)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(0))[:48].sort().values.cuda()
    r = torch.zeros(48, N, device="cuda", dtype=torch.float64)
    xs = xq[rows].double()
    for gi in range(K // 64):
        part = xs[:, gi * 64:(gi + 1) * 64] @ wq[:, gi * 64:(gi + 1) * 64].double().t()
        r += part * sxT[gi, rows].double()[:, None]
    r *= sw.double()[None, :]
    e_ours = ((y[rows].double() - r).norm() / r.norm()).item()
    e_round = ((r.to(torch.bfloat16).double() - r).norm() / r.norm()).item()
    assert e_ours <= 1.05 * e_round + 1e-6, (e_ours, e_round)
    ref = oracle.gemm_i8_grouped(xq[rows].cpu().numpy(), sxT[:, rows].cpu().numpy().copy(), wq.cpu().numpy(),
                                 sw.cpu().numpy())
    assert np.array_equal(host_bits(y[rows]), ref)


@pytest.mark.parametrize("form", ["default", "seq"])
@pytest.mark.parametrize("M,K,N,bias,gelu", [(300, 1152, 1152, True, False), (65, 2048, 3072, False, True),
                                             (17, 256, 192, True, True), (129, 4352, 4352, False, False)])
def test_gemm_i8_q_equals_gemm_then_quant_groups(E, M, K, N, bias, gelu, form, tune):
    """The INT8-output form (its row maxima, scales and bytes) against gemm_i8 + grouped quant_rows, on the automatic
    kernel and on the 128 x 128 tile-sequential fold."""
    if form == "seq":
        tune("LFM2Q_GEMM_BM", "128")
        tune("LFM2Q_GEMM_BN", "128")
        tune("LFM2Q_GEMM_GSEQ", "1")
    xq, sxT, wq, sw, b = operands(M * 3 + N, M, K, N, bias)
    y = run_grouped(E, xq, sxT, wq, sw, b, gelu)
    rq = torch.empty(M, N, device="cuda", dtype=torch.int8)
    rs = torch.empty(N // 64, M, device="cuda")
    E.quant_rows(y, rq, rs)
    q = torch.empty_like(rq)
    s = torch.empty_like(rs)
    E.gemm_i8_q(dev(xq), dev(sxT), dev(wq), dev(sw), None if b is None else dev_bf16(b), q, s, gelu)
    assert torch.equal(q, rq) and torch.equal(s, rs), f"q mismatches {(q != rq).sum().item()}"


def test_int8_linear_grouped_and_quant_out(cuda, monkeypatch):
    """Int8Linear's default (grouped-64 activation scales) and quant_out path, against the ops by hand."""
    monkeypatch.delenv("LFM2_INT8_GROUP", raising=False)
    from lfm2opt.int8 import Int8Linear, quantize_rows
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    g = torch.Generator(device="cuda").manual_seed(4)
    w = (torch.randn(256, 1152, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(256, device="cuda", generator=g).to(torch.bfloat16)
    x = torch.randn(3, 50, 1152, device="cuda", generator=g).to(torch.bfloat16)
    lin = Int8Linear(w, b)
    assert lin.group == 64
    y = lin(x)
    xq, sx = quantize_rows(x.reshape(-1, 1152), 64)
    ref = torch.empty(150, 256, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(xq, sx, lin.q, lin.s, b, ref, False)
    assert torch.equal(y.reshape(150, 256), ref)
    yq, ys = lin(x, gelu=True, quant_out=True)
    rq, rs = torch.empty_like(yq), torch.empty_like(ys)
    E.gemm_i8_q(xq, sx, lin.q, lin.s, b, rq, rs, True)
    assert torch.equal(yq, rq) and torch.equal(ys, rs)


def test_grouped_argument_errors(E):
    xq = torch.zeros(4, 128, device="cuda", dtype=torch.int8)
    w = torch.zeros(96, 128, device="cuda", dtype=torch.int8)
    sxT, sw = torch.ones(2, 4, device="cuda"), torch.ones(96, device="cuda")
    yq, ys = torch.empty(4, 96, device="cuda", dtype=torch.int8), torch.empty(1, 4, device="cuda")
    with pytest.raises(RuntimeError, match=r"w \[N, K\] with N % 64 == 0"):
        E.gemm_i8_q(xq, sxT, w, sw, None, yq, ys, False)
    w64, sw64 = w[:64].contiguous(), sw[:64].contiguous()
    yq64 = torch.empty(4, 64, device="cuda", dtype=torch.int8)
    with pytest.raises(RuntimeError, match="sxT shape"):
        E.gemm_i8_q(xq, torch.ones(4, device="cuda"), w64, sw64, None, yq64, ys, False)
    with pytest.raises(RuntimeError, match="yq / ysT shape"):
        E.gemm_i8_q(xq, sxT, w64, sw64, None, yq64, torch.empty(2, 4, device="cuda"), False)
    torch.cuda.synchronize()
