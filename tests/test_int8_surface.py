"""The W8A8 / W8A16 Python surface of lfm2opt.int8 on the CPU: the environment rules of act_group and a16_kinds
(src/lfm2opt/int8.py:22-36), scale buffer shapes (qbuf) and Int8Linear's construction (padding, quantized weights,
argument errors). The GPU tests run the layers against the ops called by hand."""

import pytest
import torch

from lfm2opt import int8
from lfm2opt.quant import quantize_int8


@pytest.fixture
def env(monkeypatch):
    for v in ("LFM2_INT8_GROUP", "LFM2_INT8_GROUP_KINDS", "LFM2_INT8_A16"):
        monkeypatch.delenv(v, raising=False)
    return monkeypatch


def test_act_group_rules(env):
    assert int8.act_group("qkv", 1152) == 64  # default: grouped
    env.setenv("LFM2_INT8_GROUP", "0")
    assert int8.act_group("qkv", 1152) == 0
    assert int8.act_group("fc2", 4304) == 64  # K > 2048 is always grouped
    assert int8.act_group("w2", 2049) == 64 and int8.act_group("w2", 2048) == 0
    env.setenv("LFM2_INT8_GROUP", "64")
    env.setenv("LFM2_INT8_GROUP_KINDS", "fc2, w2")
    assert int8.act_group("w2", 2048) == 64 and int8.act_group("qkv", 2048) == 0 and int8.act_group(None, 64) == 0
    env.setenv("LFM2_INT8_GROUP", "32")
    with pytest.raises(AssertionError):
        int8.act_group("qkv", 1152)
    env.setenv("LFM2_INT8_GROUP", "per-token")
    with pytest.raises(ValueError, match="LFM2_INT8_GROUP must be 0"):
        int8.act_group("qkv", 1152)


def test_a16_kinds(env):
    assert int8.a16_kinds() == set()
    env.setenv("LFM2_INT8_A16", "fc2,w2,")
    assert int8.a16_kinds() == {"fc2", "w2"}


def test_qbuf_shapes():
    q, s = int8.qbuf(10, 128, 0, "cpu")
    assert q.shape == (10, 128) and q.dtype == torch.int8 and s.shape == (10,) and s.dtype == torch.float32
    q, s = int8.qbuf(10, 128, 64, "cpu")
    assert s.shape == (2, 10)


def test_int8_linear_construction(env):
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(40, 100, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(40, generator=g).to(torch.bfloat16)
    lin = int8.Int8Linear(w, b, pad_n=8, pad_k=28, kind="fc1")
    assert (lin.N, lin.K) == (48, 128) and lin.group == 64
    q_ref, s_ref = quantize_int8(torch.nn.functional.pad(w, (0, 28, 0, 8)))
    assert torch.equal(lin.q, q_ref) and torch.equal(lin.s, s_ref)
    assert torch.equal(lin.bias[:40], b) and torch.equal(lin.bias[40:], torch.zeros(8, dtype=torch.bfloat16))
    pre = int8.Int8Linear(q=q_ref, scale=s_ref, a8=False)
    assert pre.q is q_ref and pre.group == 0 and pre.bias is None
    env.setenv("LFM2_INT8_GROUP", "0")
    assert int8.Int8Linear(q=q_ref, scale=s_ref, kind="qkv").group == 0
    with pytest.raises(ValueError):
        int8.Int8Linear()
    with pytest.raises(ValueError):
        int8.Int8Linear(q=q_ref)
