"""bench.py without a GPU: the one-GPU contract (--gpus above 1 exits with a message before touching a device), the
workloads it measures, and the algorithmic byte counts its GB/s and roofline figures divide by -- each checked
against the sizes of the tensors a call actually reads and writes."""

import subprocess
import sys

import pytest
import torch

from conftest import ROOT

sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

from lfm2opt.quant import quantize_int4_zp, quantize_int8  # noqa: E402


def nbytes(*ts):
    return sum(t.numel() * t.element_size() for t in ts)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("N,K,B", [(64, 128, 1), (48, 256, 5), (2048, 8192, 16)])
def test_gemv_bytes_are_the_tensors_read_and_written(N, K, B):
    W, s = quantize_int8(torch.randn(N, K))
    x, y = torch.zeros(B, K, dtype=torch.bfloat16), torch.zeros(B, N, dtype=torch.bfloat16)
    assert bench.gemv_bytes(N, K, B) == nbytes(W, s, x, y)
    assert bench.gemv_bytes(N, K, B, residual=True) == nbytes(W, s, x, y) + nbytes(y)  # the residual rows read


@pytest.mark.parametrize("S,K,B", [(32, 128, 1), (8192, 2048, 4)])
def test_swiglu_bytes_are_the_tensors_read_and_written(S, K, B):
    W, s = quantize_int8(torch.randn(2 * S, K))
    x, y = torch.zeros(B, K, dtype=torch.bfloat16), torch.zeros(B, S, dtype=torch.bfloat16)
    assert bench.swiglu_bytes(S, K, B) == nbytes(W, s, x, y)


@pytest.mark.parametrize("N,K,B,epi", [(64, 2048, 1, 0), (32, 8192, 8, 2), (2 * 256, 1024, 3, 1)])
def test_w4_bytes_are_the_gptq_tensors(N, K, B, epi):
    qw, sc, qz = quantize_int4_zp(torch.randn(N, K), bench.W4_GROUP)
    out = N // 2 if epi == 1 else N
    x, y = torch.zeros(B, K, dtype=torch.bfloat16), torch.zeros(B, out, dtype=torch.bfloat16)
    want = nbytes(qw, sc, qz, x, y) + (nbytes(y) if epi == 2 else 0)
    assert bench.w4_bytes(N, K, B, residual=epi == 2, out=out) == want


def test_workloads():
    """LFM2-1.2B: 6 attention and 10 short-conv layers; the 13 W8A8 shapes are the LM prefill projections at 512,
    2048 and 4096 tokens and the four SigLIP2 vision layers at 10240 patches (bias everywhere, GELU on fc1)."""
    assert len(bench.LAYER_TYPES) == 16 and bench.LAYER_TYPES.count("A") == 6
    shapes = {(M, K, N, bias, gelu) for M, K, N, bias, gelu, _ in bench.W8A8_SHAPES}
    lm = {(M, K, N, False, False) for M in (512, 2048, 4096) for K, N in ((2048, 3072), (2048, 16384), (8192, 2048))}
    vision = {(10240, 1152, 3456, True, False), (10240, 1152, 1152, True, False), (10240, 1152, 4304, True, True),
              (10240, 4304, 1152, True, False)}
    assert len(bench.W8A8_SHAPES) == 13 and shapes == lm | vision


def test_unknown_prefill_configuration_is_refused_before_building_the_model():
    with pytest.raises(ValueError, match="unknown prefill configuration"):
        bench.prefill_e2e_results(only="int8.1000")
