"""PyTorch-CPU restatements of the reference's dequant-matmul references, timed by bench.py as the CPU baseline.

TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg). Each expression is the reference test's own reference
computation, evaluated on the host cores.
"""

import torch
import torch.nn.functional as F


def gemv_w8_dequant_matmul(Wq, scale, x):
    """tests/test_kernels.py:137: F.linear(x.float(), Wq.float() * scale[:, None]).to(bf16), dequant included."""
    return F.linear(x.float(), Wq.float() * scale[:, None]).to(torch.bfloat16)


def gemv_w4_dequant_matmul(q, S, Z, x, group):
    """tests/test_kernels.py:150 with the zero-point format: w = s (q - z), q/z unpacked int [N, K] / [N, G]."""
    w = (q.float() - Z.float().repeat_interleave(group, 1)) * S.float().repeat_interleave(group, 1)
    return F.linear(x.float(), w).to(torch.bfloat16)


def w8a8_fake_quant(x, wq, sw, bias=None, gelu=False):
    """Per-token quant (tests/test_int8_gemm.py:35-38) then the fake-quant product of
    profiling/int8_quality_probe.py:150-160: (xq.float() * sx) @ (wq.float() * sw).T (+ b) (GELU) -> bf16."""
    xf = x.float()
    a = xf.abs().amax(-1).clamp_min(1e-8)
    sx = a / torch.full_like(a, 127.0)
    xq = torch.round(xf / sx[:, None]).clamp(-127, 127)
    y = (xq * sx[:, None]) @ (wq.float() * sw[:, None]).t()
    if bias is not None:
        y = y + bias.float()
    if gelu:
        y = F.gelu(y, approximate="tanh")
    return y.to(torch.bfloat16)
