"""Weight formats of lfm2opt.quant (CPU): closed forms, round trips, and agreement of the packed layouts with the
bit layouts the oracle and the kernels read (src/lfm2opt/quant.py:13-47, src/lfm2opt/gptq.py:164-169; the round
trip mirrors tests/test_gptq.py:47-49 of the reference)."""

import importlib.util

import numpy as np
import torch

import oracle
from conftest import GOLDEN
from lfm2opt import quant

_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)

G = torch.Generator().manual_seed(0)


def test_quantize_int8_closed_form():
    w = torch.randn(40, 256, generator=G) * 0.05
    w[3] = 0.0  # all-zero row: the 1e-12 floor keeps the scale finite, q = 0
    q, s = quant.quantize_int8(w)
    assert q.dtype == torch.int8 and s.dtype == torch.float32
    amax = w.abs().amax(1)
    assert torch.equal(s, (amax / 127).clamp_min(1e-12))
    assert int(q.abs().max()) <= 127 and torch.equal(q[3], torch.zeros(256, dtype=torch.int8))
    # the row maximum maps to +-127 and every element is within half a step of its dequantized value
    assert torch.equal(q.abs().amax(1)[amax > 0], torch.full(((amax > 0).sum(),), 127, dtype=torch.int8))
    assert ((q.float() * s[:, None] - w).abs() <= s[:, None] * 0.5 * (1 + 1e-6)).all()


def test_quantize_int4_symmetric_layout_and_round_trip():
    N, K, group = 12, 512, 128
    w = torch.randn(N, K, generator=G) * 0.02
    packed, s = quant.quantize_int4(w, group)
    assert packed.shape == (N, K // 2) and packed.dtype == torch.uint8 and s.shape == (N, K // group)
    # unpack independently: weight 2j in the low nibble of byte j, stored as q + 8
    p = packed.numpy()
    q = np.empty((N, K), np.int64)
    q[:, 0::2], q[:, 1::2] = (p & 15).astype(np.int64) - 8, (p >> 4).astype(np.int64) - 8
    assert q.min() >= -8 and q.max() <= 7
    assert np.array_equal(make_golden.pack_ref_int4(q), p)
    deq = quant.dequantize_int4(packed, s)
    assert torch.equal(deq, torch.from_numpy(q).float().view(N, K // group, group).mul(s[..., None]).view(N, K))
    assert ((deq - w).abs().view(N, K // group, group) <= s[..., None] * 0.5 * (1 + 1e-6)).all()
    # pack_int4 of the dequantized weights reproduces the packed bytes exactly
    p2, s2 = quant.pack_int4(deq, s)
    assert torch.equal(p2, packed) and torch.equal(s2, s)


def test_symmetric_bytes_are_the_int32_nibble_layout():
    """Read as little-endian int32 words, the uint8 [N, K/2] bytes are [N, K/8] with nibble i of word w = k 8w+i."""
    q = np.random.default_rng(1).integers(-8, 8, (4, 64))
    words = make_golden.pack_ref_int4(q).view("<i4")
    assert np.array_equal(words, make_golden.pack_nibbles(q + 8))


def test_quantize_int4_zp_layout_and_error_bound():
    N, K, group = 10, 1024, 128
    w = torch.randn(N, K, generator=G) * 0.03 + 0.01
    qw, s, qz = quant.quantize_int4_zp(w, group)
    Gn = K // group
    assert qw.shape == (N, K // 8) and qw.dtype == torch.int32
    assert s.shape == (N, Gn) and s.dtype == torch.float16 and qz.shape == (N, (Gn + 7) // 8)
    wv = qw.numpy().view(np.uint32)
    q = np.stack([(wv >> (4 * i)) & 15 for i in range(8)], -1).reshape(N, K).astype(np.int64)
    zv = qz.numpy().view(np.uint32)
    z = np.stack([(zv >> (4 * i)) & 15 for i in range(8)], -1).reshape(N, -1)[:, :Gn].astype(np.int64)
    assert np.array_equal(make_golden.pack_nibbles(q), qw.numpy())
    assert np.array_equal(make_golden.pack_nibbles(z), qz.numpy())
    sf = s.float().numpy().astype(np.float64)
    deq = quant.dequantize_int4_zp(qw, s, qz).numpy().astype(np.float64)
    expect = (q.reshape(N, Gn, group) - z[..., None]) * sf[..., None]
    assert np.allclose(deq, expect.reshape(N, K), rtol=0, atol=1e-7)
    # asymmetric min/max quantization: within half a step, plus the fp16 rounding of the scale
    err = np.abs(deq - w.numpy().astype(np.float64)).reshape(N, Gn, group)
    assert (err <= sf[..., None] * 0.5 + 16 * np.abs(sf[..., None]) * 2.0 ** -10).all()


def test_oracle_gemv_w4z_reads_the_packed_layout():
    N, K, group = 6, 512, 128
    w = torch.randn(N, K, generator=G) * 0.02
    qw, s, qz = quant.quantize_int4_zp(w, group)
    x = oracle.f2bf(np.random.default_rng(2).standard_normal((1, K)).astype(np.float32))
    y = oracle.gemv_w4z(qw.numpy(), s.numpy(), qz.numpy(), x, group)
    deq = quant.dequantize_int4_zp(qw, s, qz).double().numpy()
    exact = oracle.bf2f(x).astype(np.float64) @ deq.T
    got = oracle.bf2f(y).astype(np.float64)
    assert np.all(np.abs(got - exact) <= np.abs(exact) * 2.0 ** -8 + 1e-6)


def _int4_sq_err(wg, s):
    """fp64 squared error of the symmetric INT4 reconstruction of each group with scale s (brute force)."""
    q = np.clip(np.round(wg / s[..., None]), -8, 7)
    return ((q * s[..., None] - wg) ** 2).sum(-1)


def test_quantize_int4_clip_search_brute_force():
    """clip_search (src/lfm2opt/quant.py:23-35): per group the chosen scale is one of the 16 candidates amax * a / 7,
    a in linspace(0.70, 1.00, 16), and no candidate reconstructs the group with a smaller squared error (checked in
    fp64 over every candidate); groups with one large outlier pick a clipped scale (a < 1); the packed weights are
    round(w / s) of the chosen scale; without the search the scale stays amax / 7."""
    N, K, group = 6, 512, 128
    w = torch.randn(N, K, generator=G) * 0.02
    w[1, 5] = 0.5   # outliers: clipping the rest of the group lowers the error
    w[4, 300] = -0.4
    packed, s = quant.quantize_int4(w, group, True)
    _, s_plain = quant.quantize_int4(w, group, False)
    wg = w.double().numpy().reshape(N, K // group, group)
    amax = np.maximum(np.abs(w.float().numpy().reshape(N, K // group, group)).max(-1), 1e-12).astype(np.float32)
    fr = torch.linspace(0.70, 1.00, 16).numpy()
    cands = np.stack([amax * np.float32(a) / np.float32(7) for a in fr])        # fp32 arithmetic, as the search
    errs = np.stack([_int4_sq_err(wg, c.astype(np.float64)) for c in cands])   # [16, N, G]
    sn = s.numpy()
    chosen = (cands == sn[None]).argmax(0)
    assert ((cands == sn[None]).any(0)).all(), "scale is not one of the candidates"
    best = errs.min(0)
    got = np.take_along_axis(errs, chosen[None], 0)[0]
    assert (got <= best * (1 + 1e-6) + 1e-18).all()
    assert chosen[1, 0] < 15 and chosen[4, 2] < 15  # the outlier groups are clipped
    assert torch.equal(s_plain, (w.abs().view(N, -1, group).amax(-1).clamp_min(1e-12) / 7))
    p = packed.numpy().astype(np.int64)
    q = np.empty((N, K), np.int64)
    q[:, 0::2], q[:, 1::2] = (p & 15) - 8, (p >> 4) - 8
    ref = np.clip(np.round(w.numpy().reshape(N, -1, group) / sn[..., None]), -8, 7).reshape(N, K)
    assert np.array_equal(q, ref)


def test_quantize_int4_clip_search_row_chunks():
    """The search runs over row chunks: a matrix larger than one chunk gives the rows of the chunked and the
    one-chunk searches the same scales."""
    w = torch.randn(2 * quant.CLIP_ROWS + 3, 256, generator=G) * 0.02
    _, s_all = quant.quantize_int4(w, 128, True)
    for r0 in (0, quant.CLIP_ROWS - 1, 2 * quant.CLIP_ROWS):
        _, s_part = quant.quantize_int4(w[r0:r0 + 2], 128, True)
        assert torch.equal(s_all[r0:r0 + 2], s_part)
