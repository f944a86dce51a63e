"""W8A8 GEMM and per-token activation quantization on the GPU (through the C ABI via lfm2opt.kernels.int8_ext())
against the CPU oracle and, at the full prefill / vision shapes, against exact fp64 products on the GPU.

Parity bar (tests/test_int8_gemm.py:158-175, :55-78): quantization bit-exact (q and s), int32 accumulators
bit-exact, bf16 epilogue 0 ulp without GELU and <= 1 bf16 ulp with GELU.
"""

import numpy as np
import pytest
import torch

import oracle
import rounding_cases
from conftest import GOLDEN
from gpu_util import dev, dev_bf16, host_bits, ulp_dist

pytestmark = pytest.mark.gpu

PREFILL = [(M, K, N) for M in (512, 2048, 4096) for K, N in ((2048, 3072), (2048, 16384), (8192, 2048))]
VISION = [(10240, 1152, 3456, False), (10240, 1152, 1152, False), (10240, 1152, 4304, True), (10240, 4304, 1152, False)]


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import int8_ext

    return int8_ext()


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


# ------------------------------------------------------------------------------------------------ quant_rows
@pytest.mark.parametrize("name", ["quant_rows_traps_k64", "quant_rows_m37_k1152", "quant_rows_m5_k4304",
                                  "quant_rows_m3_k8192"])
def test_quant_rows_fixture(E, name):
    f = load(name)
    rows, K = f["x"].shape
    q = torch.empty(rows, K, device="cuda", dtype=torch.int8)
    s = torch.empty(rows, device="cuda", dtype=torch.float32)
    E.quant_rows(dev_bf16(f["x"]), q, s)
    assert np.array_equal(s.cpu().numpy(), f["s"]), "scales differ"
    qq = q.cpu().numpy()
    assert np.array_equal(qq, f["q"]), f"{int((qq != f['q']).sum())} q mismatches"


@pytest.mark.parametrize("M,K", [(4096, 8192), (10240, 1152), (2048, 2048), (777, 4304), (1, 2048), (9, 96)])
def test_quant_rows_vs_oracle(E, M, K):
    """Activations ~N(0,1) with 0.1% outliers at 20 sigma (the prefill workload), every K path of the kernel."""
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g)
    out = torch.rand(M, K, generator=g) < 1e-3
    x[out] = 20.0 * torch.sign(torch.randn(int(out.sum()), generator=g))
    xb = x.to(torch.bfloat16)
    q = torch.empty(M, K, device="cuda", dtype=torch.int8)
    s = torch.empty(M, device="cuda", dtype=torch.float32)
    E.quant_rows(xb.cuda(), q, s)
    rq, rs = oracle.quant_rows(xb.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.cpu().numpy(), rq)


@pytest.mark.parametrize("wg", [0, 1])
@pytest.mark.parametrize("M,K", [(512, 8192), (512, 2048), (777, 4304), (3, 1024), (2048, 6144), (10240, 1152)])
def test_quant_both_kernels_vs_oracle(E, tune, wg, M, K):
    """quant_rows and grouped quant_rows on each of the two launch forms (a wavefront per row, LFM2Q_QUANT_WG=0, and
    a workgroup per row, =1): q and s bit-exact against the oracle, 0.1% outliers at 20 sigma, K with a partial last
    vector round (4304 = 538 vectors over 256 threads), the golden division traps in row 0."""
    tune("LFM2Q_QUANT_WG", wg)
    g = torch.Generator().manual_seed(M * 7 + K)
    x = torch.randn(M, K, generator=g)
    out = torch.rand(M, K, generator=g) < 1e-3
    x[out] = 20.0 * torch.sign(torch.randn(int(out.sum()), generator=g))
    xb = x.to(torch.bfloat16)
    bits = xb.view(torch.int16).numpy().view(np.uint16).copy()
    traps = load("quant_rows_traps_k64")["x"][0]
    bits[0, :traps.size] = traps
    xd = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
    q = torch.empty(M, K, device="cuda", dtype=torch.int8)
    s = torch.empty(M, device="cuda", dtype=torch.float32)
    E.quant_rows(xd, q, s)
    rq, rs = oracle.quant_rows(bits)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.cpu().numpy(), rq)
    if K % 64 == 0:
        sT = torch.empty(K // 64, M, device="cuda", dtype=torch.float32)
        E.quant_rows(xd, q, sT)
        gq, gs = oracle.quant_groups(bits)
        assert np.array_equal(sT.cpu().numpy(), gs)
        assert np.array_equal(q.cpu().numpy(), gq)


# ------------------------------------------------------------------------------------------------ fixtures
@pytest.mark.parametrize("name", ["gemm_i8_m37_k320_n24_bias", "gemm_i8_m70_k1152_n100",
                                  "gemm_i8_m33_k576_n40_bias_gelu", "gemm_i8_m129_k4304_n72_bias"])
def test_gemm_fixture(E, name):
    f = load(name)
    M, N = f["y"].shape
    xq, wq = dev(f["xq"]), dev(f["wq"])
    c = torch.empty(M, N, device="cuda", dtype=torch.int32)
    E.gemm_i8_i32(xq, wq, c)
    assert np.array_equal(c.cpu().numpy(), f["acc"]), "int32 accumulators differ"
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    gelu = "gelu" in name
    E.gemm_i8(xq, dev(f["sx"]), wq, dev(f["sw"]), dev_bf16(f["bias"]) if "bias" in f else None, y, gelu)
    u = int(ulp_dist(host_bits(y), f["y"]).max())
    assert u <= (1 if gelu else 0), f"{u} bf16 ulp"


# ------------------------------------------------------------------------------------------------ seeded parity
def _operands(seed, M, K, N, bias):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    xq, sx = oracle.quant_rows(x.view(torch.int16).numpy().view(np.uint16))
    wq, sw = oracle.quant_rows(w.view(torch.int16).numpy().view(np.uint16))
    b = (torch.randn(N, generator=g).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)) if bias else None
    return xq, sx, wq, sw, b


@pytest.mark.parametrize("M,K,N,bias,gelu", [(272, 2048, 3072, False, False), (17, 2048, 2048, False, False),
                                             (1, 1152, 1152, True, False), (300, 1152, 1152, True, True),
                                             (257, 4304, 1152, True, False), (64, 1152, 4304, True, True)])
def test_gemm_vs_oracle(E, M, K, N, bias, gelu):
    """The reference test's shapes (tests/test_int8_gemm.py:256-259, scaled to oracle-friendly M) plus the vision
    fc2 K = 4304 and fc1 N = 4304 tails."""
    xq, sx, wq, sw, b = _operands(M * 7 + N, M, K, N, bias)
    acc = oracle.gemm_i8_i32(xq, wq)
    ref = oracle.gemm_i8_epilogue(acc, sx, sw, b, gelu)
    c = torch.empty(M, N, device="cuda", dtype=torch.int32)
    E.gemm_i8_i32(dev(xq), dev(wq), c)
    assert np.array_equal(c.cpu().numpy(), acc)
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(dev(xq), dev(sx), dev(wq), dev(sw), None if b is None else dev_bf16(b), y, gelu)
    u = int(ulp_dist(host_bits(y), ref).max())
    assert u <= (1 if gelu else 0), f"{u} bf16 ulp"


def _bf16a_vs_pair(E, x, w, sw, b, gelu):
    """gemm_i8_bf16a(x) against quant_rows(x) + gemm_i8: the scales and every output bit for bit."""
    M, K = x.shape
    N = w.shape[0]
    xq = torch.empty(M, K, device="cuda", dtype=torch.int8)
    s = torch.empty(M, device="cuda")
    y1 = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.quant_rows(x, xq, s)
    E.gemm_i8(xq, s, w, sw, b, y1, gelu)
    s2 = torch.full((M,), -1.0, device="cuda")
    y2 = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8_bf16a(x, s2, w, sw, b, y2, gelu)
    torch.cuda.synchronize()
    assert torch.equal(s2, s), "scales differ from quant_rows'"
    assert torch.equal(y2.view(torch.int16), y1.view(torch.int16)), \
        f"{int((y2.view(torch.int16) != y1.view(torch.int16)).sum())} outputs differ from quant_rows + gemm_i8"


@pytest.mark.parametrize("tile", [None, (128, 128), (128, 64), (64, 128), (64, 64)])
@pytest.mark.parametrize("M,K,N,bias,gelu", [(70, 1152, 96, True, True), (129, 4304, 72, True, False),
                                             (1, 16, 8, False, False), (300, 2048, 3072, False, False),
                                             (513, 8192, 2048, False, False), (64, 64, 1000, True, True)])
def test_gemm_bf16a_equals_quant_then_gemm(E, M, K, N, bias, gelu, tile, tune):
    """bf16 activations quantized inside the GEMM: ragged M / N / K tails, every tile, K from one stage to 128
    stages; activations ~N(0,1) with 0.1 % outliers at 20 sigma."""
    if tile:
        tune("LFM2Q_GEMM_BM", tile[0])
        tune("LFM2Q_GEMM_BN", tile[1])
    g = torch.Generator(device="cuda").manual_seed(M * 3 + K + N)
    x = torch.randn(M, K, device="cuda", generator=g)
    x = torch.where(torch.rand(M, K, device="cuda", generator=g) < 1e-3, 20.0 * torch.sign(x), x).to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
    _bf16a_vs_pair(E, x, w, sw, b, gelu)


def test_gemm_bf16a_division_traps(E):
    """The golden rows whose values sit where x * (1/s) and x / s round to different integers: the in-GEMM
    quantization takes the same IEEE-division branch as quant_rows."""
    f = load("quant_rows_traps_k64")
    x = dev_bf16(f["x"])
    M, K = x.shape
    g = torch.Generator(device="cuda").manual_seed(3)
    w = torch.randint(-127, 128, (40, K), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(40, device="cuda", generator=g) * 0.01 + 1e-3
    _bf16a_vs_pair(E, x, w, sw, None, False)


def test_gemm_bf16a_full_shape(E):
    """The 4096 x 2048 x 16384 prefill w1|w3 shape (128 x 128 tiles, 32 stages) against the pair, every output."""
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(4096, 2048, device="cuda", generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (16384, 2048), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(16384, device="cuda", generator=g) * 0.01 + 1e-3
    _bf16a_vs_pair(E, x, w, sw, None, False)


@pytest.mark.parametrize("tile", [None, (256, 256), (128, 64)])
def test_gemm_gelu_epilogue_over_its_input_range(E, tile, tune):
    """The GELU epilogue on ~1M distinct inputs: acc = 1 everywhere (one-hot A and B rows), so y[m, n] =
    bf16(gelu((1 * sx[m]) * sw[n] + b[n])) with sx x sw spanning [-10, 10] densely, both tails included (the
    negative tail, where 1 + tanh(u) cancels in fp32, and v > 3, where tanh(u) rounds to 1). Against the oracle's
    fp32 GELU (the reference's formula with the C library's tanhf): <= 1 bf16 ulp everywhere, and 1-ulp outputs rare
    (they can only come from fp32 values within a few ulps of a bf16 rounding boundary). Run on the persistent
    256 x 256 epilogue and on a 4-wavefront tile."""
    if tile:
        tune("LFM2Q_GEMM_BM", tile[0])
        tune("LFM2Q_GEMM_BN", tile[1])
    M, N, K = 1024, 1032, 64
    rng = np.random.default_rng(11)
    xq = np.zeros((M, K), np.int8)
    xq[:, 0] = 1
    wq = np.zeros((N, K), np.int8)
    wq[:, 0] = 1
    sx = np.sort(rng.uniform(-10.0, 10.0, M)).astype(np.float32)
    sw = rng.uniform(0.5, 1.0, N).astype(np.float32)
    b = oracle.f2bf(rng.uniform(-0.05, 0.05, N).astype(np.float32))
    ref = oracle.gemm_i8_epilogue(np.ones((M, N), np.int32), sx, sw, b, True)
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(dev(xq), dev(sx), dev(wq), dev(sw), dev_bf16(b), y, True)
    u = ulp_dist(host_bits(y), ref)
    print(f"GELU sweep: max {int(u.max())} ulp, {int((u > 0).sum())} of {u.size} outputs at 1 ulp")
    assert int(u.max()) <= 1
    assert (u > 0).sum() <= 1e-3 * u.size


def _full_check(E, M, K, N, bias, gelu, seed):
    """Full-size GEMM: int32 against an exact fp64 product on the GPU, bf16 output of 256 sampled rows against the
    reference test's fp32 epilogue expression (tests/test_int8_gemm.py:166-172) evaluated by torch on the GPU."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    xq = torch.randint(-127, 128, (M, K), device="cuda", dtype=torch.int8, generator=g)
    wq = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    sx = torch.rand(M, device="cuda", generator=g) * 0.05 + 1e-3
    sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
    c = torch.empty(M, N, device="cuda", dtype=torch.int32)
    E.gemm_i8_i32(xq, wq, c)
    exact = (xq.double() @ wq.double().t())
    assert torch.equal(c.double(), exact), "int32 accumulators differ from the exact product"
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(xq, sx, wq, sw, b, y, gelu)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(seed))[:256].cuda()
    r = exact[rows].float() * sx[rows, None]
    r = r * sw[None, :]
    if b is not None:
        r = r + b.float()
    if gelu:
        r = torch.nn.functional.gelu(r, approximate="tanh")
    u = int(ulp_dist(host_bits(y[rows]), host_bits(r.to(torch.bfloat16))).max())
    assert u <= (1 if gelu else 0), f"{u} bf16 ulp"


@pytest.mark.parametrize("M,K,N", PREFILL)
def test_gemm_prefill_shapes(E, M, K, N):
    _full_check(E, M, K, N, False, False, M + K + N)


@pytest.mark.parametrize("M,K,N,gelu", VISION)
def test_gemm_vision_shapes(E, M, K, N, gelu):
    _full_check(E, M, K, N, True, gelu, K + N)


TILES = [(256, 256), (128, 256), (256, 128), (128, 128), (128, 64), (64, 128), (64, 64)]


_PERS = [(256, 256), (256, 128), (128, 128), (128, 64)]
EVERY_CONFIG = ([dict(BM=bm, BN=bn, STAGES=3, KSPLIT=1, BIGP=0) for bm, bn in TILES]
                + [dict(BM=bm, BN=bn, STAGES=6, KSPLIT=1, BIGP=0) for bm, bn in TILES if bm + bn <= 384]
                + [dict(BM=bm, BN=bn, STAGES=3, KSPLIT=2, BIGP=0) for bm, bn in TILES if bm + bn <= 384]
                + [dict(BM=bm, BN=bn, STAGES=3, KSPLIT=4, BIGP=0) for bm, bn in TILES if bm + bn <= 192]
                + [dict(BM=bm, BN=bn, BIGP=1, SPLITK=1) for bm, bn in _PERS]
                + [dict(BM=bm, BN=bn, BIGP=1, SPLITK=sk) for bm, bn in _PERS[1:] for sk in (2, 4)]
                + [dict(BM=256, BN=256, BIGP=0, RING=r) for r in (1282, 644, 645)])


@pytest.mark.parametrize("M,K,N,bias,gelu", [(M, K, N, False, False) for M, K, N in PREFILL]
                         + [(M, K, N, True, g) for M, K, N, g in VISION])
def test_gemm_every_configuration_full_shapes(E, M, K, N, bias, gelu, tune):
    """Every forced per-token configuration (tile, ring depth, in-workgroup K split, persistent or one workgroup per
    tile, K split across workgroups, the 256 x 256 ring forms) at the full prefill / vision shapes, on quantized
    ~N(0,1) activations with 0.1 % outliers at 20 sigma, two calls each: bit-identical to the automatic choice, which
    equals hipBLASLt's exact int32 product (torch._int_mm) followed by the epilogue as separate fp32 torch ops (0 ulp;
    with GELU the same check runs without it, and the GELU outputs are compared across configurations); and the
    int32-output kernel of every tile equals torch._int_mm."""
    g = torch.Generator(device="cuda").manual_seed(M + K + N)
    wq = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
    b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
    x = torch.randn(M, K, device="cuda", generator=g)
    x[torch.rand(M, K, device="cuda", generator=g) < 1e-3] = 20.0
    xq = torch.empty(M, K, device="cuda", dtype=torch.int8)
    sx = torch.empty(M, device="cuda")
    E.quant_rows(x.to(torch.bfloat16), xq, sx)
    acc = torch._int_mm(xq, wq.t())
    r = (acc.float() * sx[:, None]) * sw[None, :]
    if bias:
        r = r + b.float()[None, :]
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(xq, sx, wq, sw, b, y, False)
    assert torch.equal(y.view(torch.int16), r.to(torch.bfloat16).view(torch.int16)), "auto vs int32 + epilogue"
    base = torch.empty_like(y)
    E.gemm_i8(xq, sx, wq, sw, b, base, gelu)
    for cfg in EVERY_CONFIG:
        for k, v in cfg.items():
            tune("LFM2Q_GEMM_" + k, str(v))
        for call in range(2):
            y.fill_(3.0)
            E.gemm_i8(xq, sx, wq, sw, b, y, gelu)
            assert torch.equal(y.view(torch.int16), base.view(torch.int16)), (cfg, call)
        for k in ("BM", "BN", "STAGES", "KSPLIT", "BIGP", "SPLITK", "RING"):
            tune("LFM2Q_GEMM_" + k, None)
    c = torch.empty(M, N, device="cuda", dtype=torch.int32)
    for bm, bn in TILES:
        tune("LFM2Q_GEMM_BM", str(bm))
        tune("LFM2Q_GEMM_BN", str(bn))
        c.fill_(7)
        E.gemm_i8_i32(xq, wq, c)
        assert torch.equal(c, acc), (bm, bn)


@pytest.mark.parametrize("bm,bn,stages,ksplit", [(bm, bn, 3, 1) for bm, bn in TILES]
                         + [(bm, bn, 6, 1) for bm, bn in TILES if bm + bn <= 384]
                         + [(bm, bn, 3, 2) for bm, bn in TILES if bm + bn <= 384]
                         + [(bm, bn, 3, 4) for bm, bn in TILES if bm + bn <= 192])
def test_gemm_every_tile_config(E, bm, bn, stages, ksplit, tune):
    """Each kernel configuration (tile forced through LFM2Q_GEMM_BM / _BN, LDS ring depth through
    LFM2Q_GEMM_STAGES, K split over 1, 2 or 4 wavefront groups through LFM2Q_GEMM_KSPLIT) on shapes with M, N and K
    tails; with a K split also K whose stages divide unevenly (1104: 18 stages) and K with fewer stages than groups
    (96: 2 stages), where some groups have nothing to add. int32 accumulators exact, bf16 epilogue bit-exact."""
    tune("LFM2Q_GEMM_BM", str(bm))
    tune("LFM2Q_GEMM_BN", str(bn))
    tune("LFM2Q_GEMM_STAGES", str(stages))
    tune("LFM2Q_GEMM_KSPLIT", str(ksplit))
    M, N = 300, 520
    for K in (4304, 1104, 96) if ksplit > 1 else (4304,):
        xq, sx, wq, sw, b = _operands(bm * 7 + bn + K, M, K, N, True)
        acc = oracle.gemm_i8_i32(xq, wq)
        c = torch.empty(M, N, device="cuda", dtype=torch.int32)
        E.gemm_i8_i32(dev(xq), dev(wq), c)
        assert np.array_equal(c.cpu().numpy(), acc), f"int32 K={K}"
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        E.gemm_i8(dev(xq), dev(sx), dev(wq), dev(sw), dev_bf16(b), y, False)
        assert int(ulp_dist(host_bits(y), oracle.gemm_i8_epilogue(acc, sx, sw, b)).max()) == 0, f"bf16 K={K}"


@pytest.mark.parametrize("tile,persistent", [pytest.param(None, None, id="auto")]
                         + [pytest.param(t, p, id=f"{t[0]}x{t[1]}-bigp{p}") for t, p in
                            [(t, "0") for t in TILES] + [(t, "1") for t in ((256, 256), (256, 128), (128, 128), (128, 64))]])
def test_gemm_epilogue_rounding_points(E, tile, persistent, tune):
    """Operands whose bf16 outputs depend on each rounding point of the per-token epilogue (tests/rounding_cases.py,
    expected bits derived by hand: fl(fl(fl(acc sx) sw) + b), no contraction), on every tile, one tile per
    workgroup and persistent."""
    if tile:
        tune("LFM2Q_GEMM_BM", str(tile[0]))
        tune("LFM2Q_GEMM_BN", str(tile[1]))
        tune("LFM2Q_GEMM_BIGP", persistent)
    xq, sx, wq, sw, b, expect = rounding_cases.per_token_epilogue_case()
    y = torch.empty(*xq.shape[:1], wq.shape[0], device="cuda", dtype=torch.bfloat16)
    E.gemm_i8(dev(xq), dev(sx), dev(wq), dev(sw), dev_bf16(b), y, False)
    y = host_bits(y)
    for (m, n), bits in expect.items():
        assert int(y[m, n]) == bits, (m, n, hex(int(y[m, n])))
    assert np.array_equal(y, oracle.gemm_i8(xq, sx, wq, sw, b))


@pytest.mark.parametrize("bm,bn", [(256, 256), (256, 128), (128, 128), (128, 64)])
@pytest.mark.parametrize("bias,gelu", [(False, False), (True, True)])
def test_gemm_persistent_big_tiles(E, bias, gelu, bm, bn, tune):
    """The persistent 256 x 256, 256 x 128, 128 x 128 and 128 x 64 kernels with more tiles than workgroups (17 x 17,
    17 x 33, 33 x 33 or 33 x 65 tiles on one workgroup per CU, so workgroups take further tiles whose first stage and
    epilogue operands load during the previous tile's epilogue), with M, N and K tails: bf16 output against the oracle's epilogue of
    the exact int32 product (bit-exact, <= 1 ulp with GELU) and bit-identical to the one-tile-per-workgroup kernel
    of the same tile (LFM2Q_GEMM_BIGP=0)."""
    tune("LFM2Q_GEMM_BM", str(bm))
    tune("LFM2Q_GEMM_BN", str(bn))
    M, K, N = 4100, 272, 4104
    xq, sx, wq, sw, b = _operands(M + N + int(gelu), M, K, N, bias)
    acc = oracle.gemm_i8_i32(xq, wq)
    ref = oracle.gemm_i8_epilogue(acc, sx, sw, b, gelu)
    outs = []
    for persistent in ("1", "0"):
        tune("LFM2Q_GEMM_BIGP", persistent)
        y = torch.full((M, N), 3.0, device="cuda", dtype=torch.bfloat16)
        E.gemm_i8(dev(xq), dev(sx), dev(wq), dev(sw), None if b is None else dev_bf16(b), y, gelu)
        outs.append(host_bits(y))
    assert int(ulp_dist(outs[0], ref).max()) <= (1 if gelu else 0)
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("bm,bn", [(256, 256), (256, 128), (128, 128), (128, 64)])
def test_gemm_big_tiles_unaligned_operands(E, bm, bn, tune):
    """Tiles of the persistent kernels with a bias view 2 bytes off a 4-byte boundary and an output view 8 bytes off
    a 16-byte one: the launcher leaves the persistent kernel (dword bias loads, 16-byte staged stores) for the
    one-tile-per-workgroup kernel's predicated path; bf16 output still bit-exact against the oracle."""
    tune("LFM2Q_GEMM_BM", str(bm))
    tune("LFM2Q_GEMM_BN", str(bn))
    M, K, N = 520, 128, 520
    xq, sx, wq, sw, b = _operands(11, M, K, N, True)
    ref = oracle.gemm_i8_epilogue(oracle.gemm_i8_i32(xq, wq), sx, sw, b, False)
    bfull = dev_bf16(np.concatenate([[0], b]).astype(np.uint16))
    yfull = torch.zeros(M * N + 4, device="cuda", dtype=torch.bfloat16)
    for bias, y in ((bfull[1:], yfull[:M * N].view(M, N)), (bfull[1:], yfull[4:].view(M, N)),
                    (dev_bf16(b), yfull[4:].view(M, N))):
        y.fill_(5.0)
        E.gemm_i8(dev(xq), dev(sx), dev(wq), dev(sw), bias, y, False)
        assert int(ulp_dist(host_bits(y), ref).max()) == 0


def _gemm_plain(xq, sx, wq, sw, b, y, gelu):
    """lfm2q_gemm_i8 (no workspace: never a K split across workgroups)."""
    from lfm2opt import _capi

    M, K = xq.shape
    _capi.call("lfm2q_gemm_i8", xq.data_ptr(), sx.data_ptr(), wq.data_ptr(), sw.data_ptr(), _capi.ptr(b), y.data_ptr(),
               M, wq.shape[0], K, int(gelu), _capi.stream(xq))


@pytest.mark.parametrize("bm,bn", [(128, 128), (256, 128), (128, 64)])
@pytest.mark.parametrize("sk", [2, 3, 4, 8])
def test_gemm_split_k_across_workgroups(E, bm, bn, sk, tune):
    """The persistent kernels with K cut into SK slices over workgroups (forced through LFM2Q_GEMM_SPLITK), the
    partial int32 tiles summed through the stream's workspace by the last workgroup of each tile: bit-identical to
    the same tile without a workspace, and to the oracle's epilogue of the exact product, on M / N / K tails (K of
    35 stages: slices of unequal length), with and without bias / GELU; three calls in a row on one workspace (the
    arrival counters must be back at 0 after each)."""
    tune("LFM2Q_GEMM_BM", str(bm))
    tune("LFM2Q_GEMM_BN", str(bn))
    for i, (M, K, N, bias, gelu) in enumerate([(300, 4432, 520, True, False), (131, 1104, 264, False, True),
                                               (300, 4432, 520, True, False)]):
        xq, sx, wq, sw, b = _operands(bm + bn + sk + i, M, K, N, bias)
        ref = oracle.gemm_i8_epilogue(oracle.gemm_i8_i32(xq, wq), sx, sw, b, gelu)
        args = [dev(xq), dev(sx), dev(wq), dev(sw), None if b is None else dev_bf16(b)]
        y0 = torch.full((M, N), 7.0, device="cuda", dtype=torch.bfloat16)
        _gemm_plain(*args, y0, gelu)
        tune("LFM2Q_GEMM_SPLITK", str(sk))
        y1 = torch.full((M, N), 9.0, device="cuda", dtype=torch.bfloat16)
        E.gemm_i8(*args, y1, gelu)
        tune("LFM2Q_GEMM_SPLITK", None)
        assert torch.equal(y0, y1), f"split {sk} differs from the unsplit kernel (call {i})"
        assert int(ulp_dist(host_bits(y1), ref).max()) <= (1 if gelu else 0)


@pytest.mark.parametrize("M,K,N", [(512, 2048, 3072), (512, 8192, 2048), (300, 8192, 2048)])
def test_gemm_split_k_automatic(E, M, K, N):
    """Shapes whose tiles leave CUs idle, where the automatic choice cuts K over workgroups: the library's call with
    the stream's workspace is bit-identical to the call without one, and the int32 product is exact."""
    xq, sx, wq, sw, b = _operands(M + K + N, M, K, N, True)
    args = [dev(xq), dev(sx), dev(wq), dev(sw), dev_bf16(b)]
    y0 = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    y1 = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    _gemm_plain(*args, y0, False)
    E.gemm_i8(*args, y1, False)
    E.gemm_i8(*args, y1, False)  # again, after the first call reset the counters
    assert torch.equal(y0, y1)
    rows = np.arange(0, M, 37)
    ref = oracle.gemm_i8_epilogue(oracle.gemm_i8_i32(xq[rows], wq), sx[rows], sw, b, False)
    assert int(ulp_dist(host_bits(y1)[rows], ref).max()) == 0


# ------------------------------------------------------------------------------------------------ errors
def test_gemm_argument_errors(E):
    xq = torch.zeros(4, 64, device="cuda", dtype=torch.int8)
    w = torch.zeros(8, 64, device="cuda", dtype=torch.int8)
    sx, sw = torch.ones(4, device="cuda"), torch.ones(8, device="cuda")
    y = torch.empty(4, 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="sx shape"):
        E.gemm_i8(xq, torch.ones(3, device="cuda"), w, sw, None, y, False)
    with pytest.raises(RuntimeError, match=r"w must be \[N, K\]"):
        E.gemm_i8(xq, sx, torch.zeros(8, 32, device="cuda", dtype=torch.int8), sw, None, y, False)
    with pytest.raises(RuntimeError, match="K % 16"):
        E.gemm_i8(torch.zeros(4, 40, device="cuda", dtype=torch.int8), sx,
                  torch.zeros(8, 40, device="cuda", dtype=torch.int8), sw, None, y, False)
    with pytest.raises(RuntimeError, match="sx shape"):  # grouped scales must be [K/64, M]
        E.gemm_i8(xq, torch.ones(2, 4, device="cuda"), w, sw, None, y, False)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        E.quant_rows(torch.zeros(2, 12, device="cuda", dtype=torch.bfloat16), torch.empty(2, 12, device="cuda",
                     dtype=torch.int8), torch.empty(2, device="cuda"))
    torch.cuda.synchronize()


def test_int8_linear_per_token(cuda, monkeypatch):
    """Int8Linear (src/lfm2opt/int8.py:54-91) with per-token scales equals quantize_rows + gemm_i8 by hand."""
    monkeypatch.setenv("LFM2_INT8_GROUP", "0")
    from lfm2opt.int8 import Int8Linear, quantize_rows
    from lfm2opt.kernels import int8_ext

    g = torch.Generator(device="cuda").manual_seed(3)
    w = (torch.randn(96, 1152, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(96, device="cuda", generator=g).to(torch.bfloat16)
    x = torch.randn(2, 5, 1152, device="cuda", generator=g).to(torch.bfloat16)
    lin = Int8Linear(w, b, kind="qkv")
    y = lin(x, gelu=True)
    assert y.shape == (2, 5, 96)
    xq, sx = quantize_rows(x.reshape(-1, 1152))
    ref = torch.empty(10, 96, device="cuda", dtype=torch.bfloat16)
    int8_ext().gemm_i8(xq, sx, lin.q, lin.s, b, ref, True)
    assert torch.equal(y.reshape(10, 96), ref)
