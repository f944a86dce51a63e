"""Every GEMV kind of the LFM2-1.2B decode step at its full shape, with the epilogue the step runs it with, in each
weight format the step is measured in: INT8 at batch 1, 4 and 16; INT4 in the reference format (uint8 + fp32
scales) and the GPTQ-style format (int32 + fp16 scales + 4-bit zero points) at batch 1 and 8. The launch path each
call takes is the automatic one (at these shapes: the batch-1 one-shot and persistent kernels, the matrix-core
kernels with their row-tile / K-split choices, e.g. the INT4 w1|w3 SwiGLU kernel with two row tiles at batch 8).

Each result is checked on 64 sampled output rows against the CPU oracle of that kind (gemv, gemv_swiglu,
gemv_residual, gemv_w4 / gemv_w4z with silu_mul or the bf16 residual add), to the bf16 bar max |err| / max |ref|
<= 1e-2 (mean abs error reported).
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close_bf16, host_bits

pytestmark = pytest.mark.gpu

H, FFN, VOCAB = 2048, 8192, 65536
# (kind, weight rows, K, epilogue): 0 plain, 1 SwiGLU over w1|w3 (output = rows / 2), 2 residual add
KINDS = [("qkv", 3072, H, 0), ("o+res", H, H, 2), ("in", 6144, H, 0), ("w1|w3+swiglu", 2 * FFN, H, 1),
         ("w2+res", H, FFN, 2), ("lm_head", VOCAB, H, 0)]
NSAMPLE = 64


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import ext

    return ext()


def sample_rows(nout, seed):
    return np.sort(np.random.default_rng(seed).permutation(nout)[:NSAMPLE])


def weight_rows(rows, S, epi):
    """Weight rows behind sampled output rows: for SwiGLU the w1 rows then the matching w3 rows."""
    return np.concatenate([rows, S + rows]) if epi == 1 else rows


def run_kind(fn, B, nout, epi, g):
    """(y or updated h as bf16 bits, x bits, h0 bits or None) for one launch of kind `fn(x, y)`."""
    K = fn.K
    x = torch.randn(B, K, device="cuda", generator=g).to(torch.bfloat16)
    h0 = torch.randn(B, nout, device="cuda", generator=g).to(torch.bfloat16) if epi == 2 else None
    y = h0.clone() if epi == 2 else torch.empty(B, nout, device="cuda", dtype=torch.bfloat16)
    fn(x, y)
    return host_bits(y), host_bits(x), None if h0 is None else host_bits(h0)


class Launch:
    def __init__(self, K, call):
        self.K, self.call = K, call

    def __call__(self, x, y):
        self.call(x, y)


@pytest.mark.parametrize("B", [1, 4, 16])
@pytest.mark.parametrize("kind,R,K,epi", KINDS, ids=[k[0] for k in KINDS])
def test_int8_decode_kind(E, kind, R, K, epi, B):
    g = torch.Generator(device="cuda").manual_seed(R + K + B)
    W = torch.randint(-127, 128, (R, K), device="cuda", dtype=torch.int8, generator=g)
    s = torch.rand(R, device="cuda", generator=g) * 0.01 + 1e-3
    nout = R // 2 if epi == 1 else R
    if epi == 0:
        fn = Launch(K, lambda x, y: E.gemv(W, s, x, y))
    elif epi == 1:
        fn = Launch(K, lambda x, y: E.gemv_epi(0, W, s, x, y))
    else:
        fn = Launch(K, lambda x, y: E.gemv_residual(W, s, x, y))
    out, xb, hb = run_kind(fn, B, nout, epi, g)
    rows = sample_rows(nout, R + B)
    wr = torch.from_numpy(weight_rows(rows, nout, epi)).cuda()
    Wn, sn = W[wr].cpu().numpy(), s[wr].cpu().numpy()
    if epi == 0:
        ref = oracle.gemv(Wn, sn, xb)
    elif epi == 1:
        ref = oracle.gemv_swiglu(Wn, sn, xb)
    else:
        ref = oracle.gemv_residual(Wn, sn, xb, np.ascontiguousarray(hb[:, rows]))
    assert_close_bf16(out[:, rows], ref, what=f"int8 {kind} B={B} sampled rows vs oracle")


def _w4_weights(fmt, R, K, g, group=128):
    G = K // group
    if fmt == 0:
        Wp = torch.randint(0, 256, (R, K // 2), device="cuda", dtype=torch.uint8, generator=g)
        S = torch.randn(R, G, device="cuda", generator=g).abs() * 0.02 + 1e-3
        return Wp, S, None
    Wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (R, K // 8), device="cuda", dtype=torch.int32, generator=g)
    S = (torch.randn(R, G, device="cuda", generator=g).abs() * 0.02 + 1e-3).half()
    Z = torch.randint(-2 ** 31, 2 ** 31 - 1, (R, (G + 7) // 8), device="cuda", dtype=torch.int32, generator=g)
    return Wq, S, Z


@pytest.mark.parametrize("B", [1, 8])
@pytest.mark.parametrize("fmt", [0, 1], ids=["ref-format", "gptq-format"])
@pytest.mark.parametrize("kind,R,K,epi", KINDS, ids=[k[0] for k in KINDS])
def test_int4_decode_kind(E, kind, R, K, epi, fmt, B):
    g = torch.Generator(device="cuda").manual_seed(R + K + B + 17 * fmt)
    Wt, S, Z = _w4_weights(fmt, R, K, g)
    nout = R // 2 if epi == 1 else R
    if fmt == 0:
        fn = Launch(K, lambda x, y: E.gemv_w4(Wt, S, x, y, 0, epi))
    else:
        fn = Launch(K, lambda x, y: E.gemv_w4z(Wt, S, Z, x, y, epi))
    out, xb, hb = run_kind(fn, B, nout, epi, g)
    rows = sample_rows(nout, R + B + fmt)
    wr = torch.from_numpy(weight_rows(rows, nout, epi)).cuda()
    if fmt == 0:
        plain = oracle.gemv_w4(Wt[wr].cpu().numpy(), S[wr].cpu().numpy(), xb)
    else:
        plain = oracle.gemv_w4z(Wt[wr].cpu().numpy(), S[wr].cpu().numpy(), Z[wr].cpu().numpy(), xb, 128)
    if epi == 0:
        ref = plain
    elif epi == 1:  # the oracle's fused SwiGLU for the GPTQ-style format, silu_mul of the plain GEMV otherwise
        ref = (oracle.gemv_w4z(Wt[wr].cpu().numpy(), S[wr].cpu().numpy(), Z[wr].cpu().numpy(), xb, 128, swiglu=True)
               if fmt == 1 else oracle.silu_mul(plain))
    else:
        ref = oracle.f2bf(oracle.bf2f(np.ascontiguousarray(hb[:, rows])) + oracle.bf2f(plain))
    assert_close_bf16(out[:, rows], ref, what=f"int4 fmt {fmt} {kind} B={B} sampled rows vs oracle")
