"""The decode dispatch (lfm2opt.decode.DecodeLinears, the reference's StaticDecoder._linear and its fused SwiGLU call
site, src/lfm2opt/runtime.py:218-244,277-282) on the GPU against the CPU oracle.

Each call is checked against the oracle of the path that ran: the GEMV oracles on the stored INT8 / INT4 / BF16
weights, the W8A16 oracle for the INT8-weight GEMM, and the fp64 product with the BF16 weight for F.linear. Parity
bar: bf16 outputs within max |err| / max |ref| <= 1e-2. The path taken must be the one linear_path names, and the
batch sizes are chosen so that every path runs: the GEMV (batch 1, 2..16, chunked above 16), W8A16 and F.linear.
AWQ: the GEMV must run on bf16(x * bf16(inv_s)) (runtime.py:239-240) while the kept BF16 copy takes x as it is.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close_bf16, dev_bf16, host_bits

pytestmark = pytest.mark.gpu

# (N, K): narrow, the stacked w1|w3, K = 8192 (the w2 rule), 8192 rows (the w1|w3-sized rule) and 32768 rows (the
# lm_head rule)
SHAPES = {("qkv", 0): (384, 512), ("w13", 0): (640, 512), ("w2", 0): (128, 8192), ("w13", 1): (8192, 256),
          ("head", 0): (32768, 256)}


@pytest.fixture(scope="module")
def weights(cuda):
    g = torch.Generator(device="cuda").manual_seed(5)
    return {k: (torch.randn(n, kk, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
            for k, (n, kk) in SHAPES.items()}


def make(weights, mode, **kw):
    from lfm2opt.decode import DecodeLinears

    return DecodeLinears(weights, gemv=mode, **kw)


def np_(t):
    return t.detach().cpu().numpy()


def x_for(B, K, seed):
    return oracle.f2bf(np.random.default_rng(seed).standard_normal((B, K)).astype(np.float32))


def prescale(x, inv_s):
    """bf16(x * bf16(inv_s)): the product of two bf16 values is exact in fp32, so this is torch's bf16 multiply."""
    return oracle.f2bf(oracle.bf2f(x) * oracle.bf2f(oracle.f2bf(np_(inv_s).astype(np.float32))))


def oracle_linear(D, key, path, x):
    """The oracle of the path that ran, on the weights that path reads."""
    if path == "linear":
        return oracle.gemv(host_bits(D._bf16_weight(key)), None, x)
    w = D.lin[key]
    if path == "w8a16":
        return oracle.gemm_w8(x, np_(w), np_(D.lin_scale[key]))
    fmt = D.fmt(key)
    if fmt == "bf16":
        return oracle.gemv(host_bits(w), None, x)
    if fmt == "int8":
        return oracle.gemv(np_(w), np_(D.lin_scale[key]), x)
    if key in D.lin_inv_s:
        x = prescale(x, D.lin_inv_s[key])
    if w.dtype == torch.int32:
        S = np_(D.lin_scale[key])
        return oracle.gemv_w4z(np_(w), S, np_(D.lin_zeros[key]), x, D.shape(key)[1] // S.shape[1])
    return oracle.gemv_w4(np_(w), np_(D.lin_scale[key]), x)


def check_linear(D, key, B, seed):
    from lfm2opt.decode import linear_path

    N, K = D.shape(key)
    x = x_for(B, K, seed)
    y = D.linear(dev_bf16(x), key)
    want = linear_path(D.mode, D.fmt(key), B, N, K, key in D.lin_bf16)
    assert D.last_path == want
    assert tuple(y.shape) == (B, N)
    assert_close_bf16(host_bits(y), oracle_linear(D, key, want, x), what=f"{D.mode} {key} B={B} {want}")
    return want


@pytest.mark.parametrize("mode", ["int8", "int4", "bf16", "cublas"])
def test_linear_every_key_and_batch(weights, mode):
    D = make(weights, mode)
    seen = set()
    for B in (1, 5, 16, 24, 40):
        for key in SHAPES:
            seen.add(check_linear(D, key, B, B * 31 + len(key[0])))
    expect = {"int8": {"gemv", "linear", "w8a16"}, "int4": {"gemv", "linear"}, "bf16": {"gemv", "linear"},
              "cublas": {"linear"}}[mode]
    assert seen == expect


def test_linear_drop_bf16(weights):
    """Without BF16 copies INT8 weights take the GEMV (16-row chunks) or W8A16 above batch 16, never F.linear."""
    D = make(weights, "int8", drop_bf16=True)
    assert not D.lin_bf16
    paths = {(key, B): check_linear(D, key, B, B + 3) for key in SHAPES for B in (24, 40, 72)}
    assert paths[(("qkv", 0), 24)] == "gemv" and paths[(("qkv", 0), 40)] == "w8a16"
    assert paths[(("w2", 0), 24)] == "w8a16" and paths[(("w2", 0), 72)] == "w8a16"
    assert paths[(("head", 0), 24)] == "w8a16"
    assert paths[(("w13", 1), 24)] == "w8a16" and paths[(("w13", 0), 24)] == "gemv"


def test_linear_int8_large_batches(weights):
    """INT8 weights with a kept BF16 copy: W8A16 up to 256 rows (128 for 32768+ weight rows), F.linear beyond."""
    D = make(weights, "int8")
    assert check_linear(D, ("head", 0), 128, 7) == "w8a16" and check_linear(D, ("head", 0), 136, 8) == "linear"
    assert check_linear(D, ("qkv", 0), 256, 9) == "w8a16" and check_linear(D, ("qkv", 0), 264, 10) == "linear"


def test_keep_int8_kinds(weights):
    """w4_keep_int8: the listed kinds stay INT8 under mode "int4" (runtime.py:178) and take the INT8 paths."""
    D = make(weights, "int4", w4_keep_int8=("head", "qkv"))
    assert D.fmt(("head", 0)) == "int8" and D.fmt(("qkv", 0)) == "int8" and D.fmt(("w2", 0)) == "int4"
    assert check_linear(D, ("head", 0), 24, 1) == "w8a16"
    assert check_linear(D, ("qkv", 0), 3, 2) == "gemv"
    assert check_linear(D, ("w2", 0), 3, 3) == "gemv"


@pytest.mark.parametrize("mode", ["int8", "int4", "bf16"])
@pytest.mark.parametrize("B", [1, 7, 16, 24])
def test_swiglu_and_residual(weights, mode, B):
    """The fused GEMV epilogues on the GEMV path, the linear followed by silu_mul / a bf16 add elsewhere; both
    against the oracle's GEMV + separate op on the path's weights."""
    D = make(weights, mode)
    key = ("w13", 0)
    N, K = D.shape(key)
    x = x_for(B, K, B)
    path = D.path(B, key)
    act = D.swiglu(dev_bf16(x), key)
    assert D.last_path == path
    assert_close_bf16(host_bits(act), oracle.silu_mul(oracle_linear(D, key, path, x)),
                      what=f"{mode} swiglu B={B} {path}")
    key = ("qkv", 0)
    N, K = D.shape(key)
    x = x_for(B, K, B + 1)
    h0 = oracle.f2bf(np.random.default_rng(B).standard_normal((B, N)).astype(np.float32) * 0.5)
    path = D.path(B, key)
    h = D.residual(dev_bf16(x), key, dev_bf16(h0))
    assert D.last_path == path
    ref = oracle.f2bf(oracle.bf2f(h0) + oracle.bf2f(oracle_linear(D, key, path, x)))
    assert_close_bf16(host_bits(h), ref, what=f"{mode} residual B={B} {path}")


def test_epilogue_fusion_off_matches(weights, monkeypatch):
    """LFM2_EPI=0 (runtime.py:35): the separate GEMV + silu_mul give the same bits as the fused epilogue."""
    x = dev_bf16(x_for(4, 512, 9))
    fused = host_bits(make(weights, "int8").swiglu(x, ("w13", 0)))
    monkeypatch.setenv("LFM2_EPI", "0")
    D = make(weights, "int8")
    assert not D.epilogue_fusion
    assert np.array_equal(host_bits(D.swiglu(x, ("w13", 0))), fused)


def test_awq_prescale(weights):
    """An AWQ entry (packed, scales, inv_s): the GEMV runs on x * inv_s, the kept BF16 copy on x."""
    from lfm2opt.quant import quantize_int4

    key = ("w2", 0)
    W = weights[key]
    g = torch.Generator(device="cuda").manual_seed(11)
    s = 0.5 + 1.5 * torch.rand(W.shape[1], device="cuda", generator=g)
    packed, S = quantize_int4(W.float() * s[None, :])
    D = make(weights, "int4", w4_pre={key: (packed, S, 1.0 / s)})
    assert key in D.lin_inv_s
    assert check_linear(D, key, 3, 4) == "gemv"
    # and the GEMV on the unscaled x would differ by far more than the tolerance
    x = x_for(3, W.shape[1], 4)
    y = oracle.bf2f(host_bits(D.linear(dev_bf16(x), key)))
    unscaled = oracle.bf2f(oracle.gemv_w4(np_(packed), np_(S), x))
    assert np.abs(y - unscaled).max() / np.abs(unscaled).max() > 0.1
    assert check_linear(D, key, 24, 5) == "linear"  # BF16 copy, x as it is


def test_gptq_pre(weights):
    """A GPTQ-style entry (qweight int32, scales fp16, qzeros int32) takes gemv_w4z, alone and with inv_s."""
    from lfm2opt.quant import quantize_int4_zp

    pre = {k: quantize_int4_zp(weights[k]) for k in (("qkv", 0), ("w13", 0))}
    inv = torch.linspace(0.5, 2.0, SHAPES[("qkv", 0)][1], device="cuda")
    pre[("qkv", 0)] = pre[("qkv", 0)] + (inv,)
    D = make(weights, "int4", w4_pre=pre)
    assert D.lin[("qkv", 0)].dtype == torch.int32 and ("qkv", 0) in D.lin_inv_s
    for B in (1, 6, 16):
        assert check_linear(D, ("qkv", 0), B, B) == "gemv"
        assert check_linear(D, ("w13", 0), B, B + 50) == "gemv"
    x = x_for(6, 512, 8)
    act = D.swiglu(dev_bf16(x), ("w13", 0))
    assert_close_bf16(host_bits(act), oracle.silu_mul(oracle_linear(D, ("w13", 0), "gemv", x)), what="gptq swiglu")


def test_bad_construction(weights):
    from lfm2opt.decode import DecodeLinears

    with pytest.raises(ValueError):
        DecodeLinears(weights, gemv="int4", drop_bf16=True)
    with pytest.raises(ValueError):
        DecodeLinears({("qkv", 0): weights[("qkv", 0)].float()}, gemv="int8")
    with pytest.raises(ValueError):
        DecodeLinears(weights, gemv="int4", w4_pre={("qkv", 0): (torch.zeros(384, 100, dtype=torch.uint8,
                                                                              device="cuda"), None)})


def test_bias(weights):
    """linear(x, key, bias) on the GEMV, W8A16 and F.linear paths: y + bias within the bf16 bar."""
    D = make(weights, "int8")
    for key, B in ((("qkv", 0), 2), (("head", 0), 24), (("qkv", 0), 24)):
        N, K = D.shape(key)
        x = x_for(B, K, B + 77)
        b = oracle.f2bf(np.random.default_rng(N).standard_normal(N).astype(np.float32))
        y = D.linear(dev_bf16(x), key, dev_bf16(b))
        ref = oracle.f2bf(oracle.bf2f(oracle_linear(D, key, D.last_path, x)) + oracle.bf2f(b)[None, :])
        assert_close_bf16(host_bits(y), ref, what=f"bias {key} B={B} {D.last_path}")
