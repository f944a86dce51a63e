"""Grouped quantization and the fused INT8 producers on the GPU (through the C ABI via lfm2opt.kernels.int8_ext()).

Parity bar, following the reference's own test of these kernels (tests/test_int8_gemm.py:123-155: the fused kernel
equals the unfused bf16 kernel followed by quant_rows, exactly):
- quant_groups: q and the transposed scales bit-exact against the oracle (including the division-trap rows);
- producers: the in-place residual h = bf16(h + y) bit-exact; the bf16 row x they quantize within 1 bf16 ulp of the
  oracle (the row statistics are fp32 sums in the kernel's own order, the oracle's are fp64; 2 ulps for the rows of
  64 values, where x's two rounding points after a last-bit difference in rs both flipped once); q / s bit-identical to
  quant_rows / quant_groups of that x and to the same call without x requested; silu_mul_q's x bit-identical to
  silu_mul.
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN
from gpu_util import assert_close_bf16, dev, dev_bf16, host_bits, ulp_dist

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import int8_ext

    return int8_ext()


@pytest.fixture(scope="module")
def D(cuda):
    from lfm2opt.kernels import ext

    return ext()


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


def rand_bf16(seed, shape, scale=1.0):
    return oracle.f2bf((np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32))


def quant_of(E, x, grouped):
    """(q, s) of the bf16 tensor x by the library's standalone quantizer."""
    rows, L = x.shape
    q = torch.empty(rows, L, device="cuda", dtype=torch.int8)
    s = torch.empty((L // 64, rows) if grouped else (rows,), device="cuda")
    E.quant_rows(x, q, s)
    return q, s


def qs_buffers(rows, L, grouped):
    q = torch.empty(rows, L, device="cuda", dtype=torch.int8)
    s = torch.empty((L // 64, rows) if grouped else (rows,), device="cuda")
    return q, s


# ------------------------------------------------------------------------------------------------ quant_groups
@pytest.mark.parametrize("name", ["quant_groups_traps_k64", "quant_groups_m37_k1152"])
def test_quant_groups_fixture(E, name):
    f = load(name)
    rows, K = f["x"].shape
    q, sT = qs_buffers(rows, K, True)
    E.quant_rows(dev_bf16(f["x"]), q, sT)
    assert np.array_equal(q.cpu().numpy(), f["q"]) and np.array_equal(sT.cpu().numpy(), f["sT"])


@pytest.mark.parametrize("rows,K", [(300, 2048), (65, 4352), (3, 8192), (5, 9216)])
def test_quant_groups_vs_oracle(E, rows, K):
    x = rand_bf16(rows + K, (rows, K), 2.0)
    x[:, 100] = oracle.f2bf(np.full(rows, -60.0, np.float32))  # an outlier column
    q, sT = qs_buffers(rows, K, True)
    E.quant_rows(dev_bf16(x), q, sT)
    rq, rs = oracle.quant_groups(x)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(sT.cpu().numpy(), rs)


# ------------------------------------------------------------------------------------------------ producers
def check_x(out_x, ref_x, what, max_ulp=1):
    u = ulp_dist(out_x, ref_x)
    print(f"{what}: x max {int(u.max())} bf16 ulp, {float((u > 0).mean()):.2e} of values differ")
    assert u.max() <= max_ulp, what


@pytest.mark.parametrize("name", ["add_rmsnorm_r9_h512"])
def test_add_rmsnorm_fixture(E, name):
    f = load(name)
    h, rows, H = dev_bf16(f["h"]), *f["h"].shape
    x = torch.empty_like(h)
    q, s = qs_buffers(rows, H, False)
    E.add_rmsnorm_q(h, dev_bf16(f["y"]), dev_bf16(f["w"]), q, s, float(f["eps"]), x=x)
    assert np.array_equal(host_bits(h), f["h_out"])
    check_x(host_bits(x), f["x"], name)


@pytest.mark.parametrize("name", ["add_layernorm_r7_d1152"])
def test_add_layernorm_fixture(E, name):
    f = load(name)
    h, rows, Dm = dev_bf16(f["h"]), *f["h"].shape
    x = torch.empty_like(h)
    q, s = qs_buffers(rows, Dm, False)
    E.add_layernorm_q(h, dev_bf16(f["y"]), dev_bf16(f["w"]), dev_bf16(f["b"]), q, s, float(f["eps"]), x=x)
    assert np.array_equal(host_bits(h), f["h_out"])
    check_x(host_bits(x), f["x"], name)


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("rows,H,residual", [(257, 2048, True), (33, 1152, True), (5, 8192, False), (70, 576, True)])
def test_add_rmsnorm_q(E, rows, H, residual, grouped):
    h0, y = rand_bf16(rows, (rows, H), 2.0), rand_bf16(H, (rows, H))
    w = oracle.f2bf((np.random.default_rng(1).random(H) + 0.5).astype(np.float32))
    eps = 1e-5
    hn_ref, x_ref = oracle.add_rmsnorm(h0, y if residual else None, w, eps)
    h1, h2 = dev_bf16(h0), dev_bf16(h0)
    yd = dev_bf16(y) if residual else None
    x = torch.empty(rows, H, device="cuda", dtype=torch.bfloat16)
    q1, s1 = qs_buffers(rows, H, grouped)
    q2, s2 = qs_buffers(rows, H, grouped)
    E.add_rmsnorm_q(h1, yd, dev_bf16(w), q1, s1, eps, x=x)
    E.add_rmsnorm_q(h2, yd, dev_bf16(w), q2, s2, eps)
    assert np.array_equal(host_bits(h1), hn_ref) and torch.equal(h1, h2)
    check_x(host_bits(x), x_ref, f"add_rmsnorm_q {rows}x{H}")
    rq, rs = quant_of(E, x, grouped)
    assert torch.equal(q1, rq) and torch.equal(s1, rs) and torch.equal(q1, q2) and torch.equal(s1, s2)


@pytest.mark.parametrize("rows,H,residual,grouped", [(2563, 64, False, False), (2563, 64, True, True),
                                                    (37, 64, True, False), (13, 32, True, False), (9, 8, False, False),
                                                    (1, 64, False, True)])
def test_add_rmsnorm_q_short_rows(E, tune, rows, H, residual, grouped):
    """Rows of at most 64 values (the per-head q / k norms) run eight to a wavefront; each row equals the oracle and
    the one-row-per-wavefront kernel (LFM2Q_QUANT_WG=0) bit for bit -- h, x, q and the scales -- including a last
    wavefront only partly filled with rows."""
    h0, y = rand_bf16(rows + H, (rows, H), 2.0), rand_bf16(H + 1, (rows, H))
    w = oracle.f2bf((np.random.default_rng(3).random(H) + 0.5).astype(np.float32))
    eps = 1e-6
    hn_ref, x_ref = oracle.add_rmsnorm(h0, y if residual else None, w, eps)
    out = {}
    for form in (1, 0):
        tune("LFM2Q_QUANT_WG", form)
        hd = dev_bf16(h0)
        x = torch.empty(rows, H, device="cuda", dtype=torch.bfloat16)
        q, s = qs_buffers(rows, H, grouped)
        E.add_rmsnorm_q(hd, dev_bf16(y) if residual else None, dev_bf16(w), q, s, eps, x=x)
        out[form] = (hd, x, q, s)
    for a, b in zip(out[1], out[0]):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    assert np.array_equal(host_bits(out[1][0]), hn_ref)
    # the oracle sums the squares in double, the kernel in fp32 in its own order, so rs may differ in its last bit;
    # x = bf16(w bf16(h rs)) then has two rounding points that can each flip: 2 bf16 ulps (one value in ~160 K here)
    check_x(host_bits(out[1][1]), x_ref, f"add_rmsnorm_q short {rows}x{H}", max_ulp=2)
    rq, rs = quant_of(E, out[1][1], grouped)
    assert torch.equal(out[1][2], rq) and torch.equal(out[1][3], rs)


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("rows,Dm,residual", [(300, 1152, True), (64, 2048, False), (11, 4352, True)])
def test_add_layernorm_q(E, rows, Dm, residual, grouped):
    h0, y = rand_bf16(rows + 1, (rows, Dm), 3.0), rand_bf16(Dm + 1, (rows, Dm))
    h0[:, :5] = oracle.f2bf(oracle.bf2f(h0[:, :5]) + 6.0)  # a row mean away from zero
    r = np.random.default_rng(2)
    w, b = oracle.f2bf((r.random(Dm) + 0.5).astype(np.float32)), rand_bf16(3, (Dm,))
    eps = 1e-6
    hn_ref, x_ref = oracle.add_layernorm(h0, y if residual else None, w, b, eps)
    h1, h2 = dev_bf16(h0), dev_bf16(h0)
    yd = dev_bf16(y) if residual else None
    x = torch.empty(rows, Dm, device="cuda", dtype=torch.bfloat16)
    q1, s1 = qs_buffers(rows, Dm, grouped)
    q2, s2 = qs_buffers(rows, Dm, grouped)
    E.add_layernorm_q(h1, yd, dev_bf16(w), dev_bf16(b), q1, s1, eps, x=x)
    E.add_layernorm_q(h2, yd, dev_bf16(w), dev_bf16(b), q2, s2, eps)
    assert np.array_equal(host_bits(h1), hn_ref) and torch.equal(h1, h2)
    check_x(host_bits(x), x_ref, f"add_layernorm_q {rows}x{Dm}")
    rq, rs = quant_of(E, x, grouped)
    assert torch.equal(q1, rq) and torch.equal(s1, rs) and torch.equal(q1, q2) and torch.equal(s1, s2)


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("rows,I", [(257, 8192), (40, 1152), (3, 64)])
def test_silu_mul_q(E, D, rows, I, grouped):
    g = dev_bf16(rand_bf16(rows * I, (rows, 2 * I), 2.0))
    a = torch.empty(rows, I, device="cuda", dtype=torch.bfloat16)
    D.silu_mul(g, a)
    x = torch.empty_like(a)
    q1, s1 = qs_buffers(rows, I, grouped)
    q2, s2 = qs_buffers(rows, I, grouped)
    E.silu_mul_q(g, q1, s1, x=x)
    E.silu_mul_q(g, q2, s2)
    assert torch.equal(x, a)  # the same SwiGLU arithmetic as silu_mul
    rq, rs = quant_of(E, a, grouped)
    assert torch.equal(q1, rq) and torch.equal(s1, rs) and torch.equal(q1, q2) and torch.equal(s1, s2)
    assert_close_bf16(host_bits(a), oracle.silu_mul(host_bits(g)), what=f"silu_mul_q x {rows}x{I}")


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("rows,I", [(257, 8192), (5, 8128), (33, 4352), (9, 2048), (70, 1152), (3, 64)])
def test_silu_mul_q_workgroup_form_matches_wavefront_form(E, tune, rows, I, grouped):
    """silu_mul_q with a workgroup per row (LFM2Q_QUANT_WG=1, the default from 4096 columns) and with a wavefront per
    row (=0) give the same int8 rows, scales and bf16 x, per row and per 64-column group, on rows that do not fill
    the workgroup's last vector set."""
    g = dev_bf16(rand_bf16(rows + I, (rows, 2 * I), 2.0))
    out = {}
    for wg in (1, 0):
        tune("LFM2Q_QUANT_WG", wg)
        x = torch.empty(rows, I, device="cuda", dtype=torch.bfloat16)
        q, s = qs_buffers(rows, I, grouped)
        E.silu_mul_q(g, q, s, x=x)
        out[wg] = (q, s, x)
    for a, b in zip(out[1], out[0]):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))  # bit patterns


def test_silu_mul_q_non_grouped_length(E, D):
    """A length that is not a multiple of 64 (4304, the vision MLP width) is accepted per row, and rejected grouped."""
    rows, I = 6, 4304
    g = dev_bf16(rand_bf16(9, (rows, 2 * I)))
    a = torch.empty(rows, I, device="cuda", dtype=torch.bfloat16)
    D.silu_mul(g, a)
    q, s = qs_buffers(rows, I, False)
    E.silu_mul_q(g, q, s)
    rq, rs = quant_of(E, a, False)
    assert torch.equal(q, rq) and torch.equal(s, rs)
    assert_close_bf16(host_bits(a), oracle.silu_mul(host_bits(g)), what="silu_mul_q x 6x4304")
    with pytest.raises(RuntimeError, match="s shape"):
        E.silu_mul_q(g, q, torch.empty(I // 64, rows, device="cuda"))


def test_producer_argument_errors(E):
    h = torch.zeros(4, 512, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(512, device="cuda", dtype=torch.bfloat16)
    q, s = qs_buffers(4, 512, False)
    with pytest.raises(RuntimeError, match="w shape"):
        E.add_rmsnorm_q(h, None, torch.ones(256, device="cuda", dtype=torch.bfloat16), q, s, 1e-5)
    with pytest.raises(RuntimeError, match="y shape"):
        E.add_rmsnorm_q(h, torch.zeros(4, 256, device="cuda", dtype=torch.bfloat16), w, q, s, 1e-5)
    with pytest.raises(RuntimeError, match="q shape"):
        E.add_layernorm_q(h, None, w, w, q[:2], s, 1e-6)
    with pytest.raises(RuntimeError, match="I shape"):
        E.silu_mul_q(torch.zeros(4, 2 * 9000, device="cuda", dtype=torch.bfloat16), q, s)
    with pytest.raises(RuntimeError, match="grouped shapes"):
        E.quant_rows(h, q, torch.empty(4, 4, device="cuda"))
    torch.cuda.synchronize()
