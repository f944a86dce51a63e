"""The batch-1 GEMV that normalizes its input row itself (lfm2q_gemv_rmsnorm, through
lfm2opt.kernels.ext().gemv_rmsnorm) on the GPU.

Parity bar: bit-identical to the pair it replaces -- add_rmsnorm_q with no residual input (its bf16 x), then the
batch-1 GEMV or SwiGLU GEMV on that x -- on every batch-1 kernel form (one-shot with 1, 2 or 4 rows per wavefront,
persistent), every supported K, INT8 and BF16 weights; and the output against the oracle's RMSNorm and GEMV within
the stated bf16 tolerance (max |err| / max |ref| <= 1e-2). The rows have a wide dynamic range (0.1 % of the values at
20 sigma), so a sum of squares taken in any other order than add_rmsnorm_q's would move rs and show up as differing
bits. The decode runtime's step with the fused norms is bit-identical to the same step with add_rmsnorm_q and
separate GEMVs (LFM2_NORM_GEMV=0)."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close_bf16, host_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import ext

    return ext()


@pytest.fixture(scope="module")
def E8(cuda):
    from lfm2opt.kernels import int8_ext

    return int8_ext()


def row(g, K):
    h = torch.randn(K, generator=g) * 3.0
    out = torch.rand(K, generator=g) < 1e-3
    h[out] = 60.0 * torch.sign(torch.randn(int(out.sum()), generator=g))
    return h.to(torch.bfloat16).view(1, K).cuda()


def weights(g, R, K, int8):
    if int8:
        W = torch.randint(-127, 128, (R, K), generator=g, dtype=torch.int8).cuda()
        s = (torch.rand(R, generator=g) * 0.01 + 1e-3).cuda()
        return W, s
    return (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16).cuda(), None


def unfused(E, E8, W, s, h, nw, eps, epi):
    K = h.numel()
    x = torch.empty_like(h)
    q = torch.empty(1, K, device="cuda", dtype=torch.int8)
    sc = torch.empty(1, device="cuda")
    E8.add_rmsnorm_q(h.clone(), None, nw, q, sc, eps, x=x)
    R = W.shape[0]
    y = torch.empty(1, R // 2 if epi else R, device="cuda", dtype=torch.bfloat16)
    if epi:
        E.gemv_epi(0, W, s, x, y)
    else:
        E.gemv(W, s, x, y)
    return x, y


@pytest.mark.parametrize("int8,K", [(True, 1024), (True, 2048), (True, 4096), (True, 8192), (False, 512),
                                    (False, 2048), (False, 4096)])
@pytest.mark.parametrize("R,epi", [(3072, 0), (6144, 0), (16384, 1), (2048, 1)])
def test_gemv_rmsnorm_equals_norm_then_gemv(E, E8, int8, K, R, epi):
    g = torch.Generator().manual_seed(R + K + epi)
    W, s = weights(g, R, K, int8)
    h = row(g, K)
    nw = (torch.rand(K, generator=g) + 0.5).to(torch.bfloat16).cuda()
    eps = 1e-5
    x, ref = unfused(E, E8, W, s, h, nw, eps, epi)
    y = torch.empty_like(ref)
    h0 = h.clone()
    E.gemv_rmsnorm(W, s, h, nw, eps, y, epi)
    torch.cuda.synchronize()
    assert torch.equal(h, h0), "h was written"
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), \
        f"{int((y.view(torch.int16) != ref.view(torch.int16)).sum())} outputs differ from add_rmsnorm_q + GEMV"
    # against the oracle: its RMSNorm of h, then its GEMV (int8: scaled rows; bf16: the weights as they are)
    hb = host_bits(h)[0]
    _, x_ref = oracle.add_rmsnorm(hb[None, :], None, host_bits(nw), eps)
    assert int(np.abs(x_ref.astype(np.int64) - host_bits(x).astype(np.int64)).max()) <= 1, "x vs oracle"
    if int8 and epi == 0:
        y_ref = oracle.gemv(W.cpu().numpy(), s.cpu().numpy(), x_ref)
        assert_close_bf16(host_bits(y), y_ref, 1e-2, f"gemv_rmsnorm {R}x{K}")
    elif int8:
        y_ref = oracle.gemv_swiglu(W.cpu().numpy(), s.cpu().numpy(), x_ref)
        assert_close_bf16(host_bits(y), y_ref, 1e-2, f"gemv_rmsnorm swiglu {R}x{K}")


@pytest.mark.parametrize("form", [("LFM2Q_GEMV_PERSIST", 1), ("LFM2Q_GEMV_R", 1), ("LFM2Q_GEMV_R", 2),
                                  ("LFM2Q_GEMV_R", 4)])
@pytest.mark.parametrize("epi", [0, 1])
def test_gemv_rmsnorm_every_kernel_form(E, E8, tune, form, epi):
    """Forced batch-1 kernel forms (persistent; one-shot with 1, 2, 4 rows per wavefront) at K = 2048, a ragged row
    count: each equals the unfused pair bit for bit."""
    tune(*form)
    g = torch.Generator().manual_seed(17 + epi)
    R = 2 * 1000 + 2 if epi else 3001
    W, s = weights(g, R, 2048, True)
    h = row(g, 2048)
    nw = (torch.rand(2048, generator=g) + 0.5).to(torch.bfloat16).cuda()
    _, ref = unfused(E, E8, W, s, h, nw, 1e-6, epi)
    y = torch.empty_like(ref)
    E.gemv_rmsnorm(W, s, h, nw, 1e-6, y, epi)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_gemv_rmsnorm_argument_errors(E):
    W = torch.zeros(64, 2048, device="cuda", dtype=torch.int8)
    s = torch.ones(64, device="cuda")
    h = torch.zeros(1, 2048, device="cuda", dtype=torch.bfloat16)
    nw = torch.ones(2048, device="cuda", dtype=torch.bfloat16)
    y = torch.zeros(1, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="K in"):
        E.gemv_rmsnorm(W[:, :1536].contiguous(), s, h[:, :1536].contiguous(), nw[:1536].contiguous(), 1e-5, y)
    with pytest.raises(RuntimeError, match="batch 1"):
        E.gemv_rmsnorm(W, s, torch.zeros(2, 2048, device="cuda", dtype=torch.bfloat16), nw, 1e-5, y)
    with pytest.raises(RuntimeError, match="epi 0"):
        E.gemv_rmsnorm(W, s, h, nw, 1e-5, y, epi=2)
    with pytest.raises(RuntimeError, match="fp32 scale"):
        E.gemv_rmsnorm(W, None, h, nw, 1e-5, y)
    torch.cuda.synchronize()


def test_runtime_step_fused_norms_bit_identical(cuda, monkeypatch):
    """The decode runtime at batch 1 with every operator / FFN / final norm inside its GEMV equals the same runtime
    with add_rmsnorm_q and separate GEMVs (LFM2_NORM_GEMV=0) bit for bit: logits of 9 teacher-forced steps, graph
    replays and eager steps (hidden 1024, so every normalized linear -- qkv, in_proj, w1|w3, head -- takes the fused
    GEMV)."""
    import copy

    from lfm2_tiny import step_logits, tiny_lfm2
    from lfm2opt.runtime import StaticDecoder

    net = copy.deepcopy(tiny_lfm2(seed=5, hidden=1024, heads=8, kv_heads=2, ffn=2048)).to(cuda, torch.bfloat16)
    ids = torch.randint(0, net.config.vocab_size, (1, 9), generator=torch.Generator().manual_seed(3))
    got = {}
    for fuse in ("1", "0"):
        monkeypatch.setenv("LFM2_NORM_GEMV", fuse)
        dec = StaticDecoder(net, bucket=32, keep_logits=True, gemv="int8")
        fused = {key for key in dec.lin.lin if dec.lin.norm_fusable(1, key)}
        if fuse == "1":
            assert {"qkv", "in", "w13", "head"} <= {k[0] for k in fused}, fused
        else:
            assert not fused
        got[fuse] = (step_logits(dec, ids, graph=True), step_logits(dec, ids, graph=False))
    assert torch.equal(got["1"][0], got["1"][1]), "graph replays differ from eager steps"
    assert torch.equal(got["1"][0], got["0"][0]), "fused norms change the logits"
