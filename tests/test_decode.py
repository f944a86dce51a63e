"""The decode dispatch's path choice (lfm2opt.decode.linear_path) on the CPU: the reference's rules where they carry
over (src/lfm2opt/runtime.py:223-244: "cublas" always takes F.linear, quantized weights without a BF16 copy never
do) and the MI355X thresholds at the LFM2 decode shapes."""

import pytest

from lfm2opt.decode import linear_path

QKV, IN, W13, W2, HEAD, OUT = (3072, 2048), (6144, 2048), (16384, 2048), (2048, 8192), (65536, 2048), (2048, 2048)


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int4"])
@pytest.mark.parametrize("B", [1, 4, 16, 17, 64, 256])
def test_cublas_mode_is_always_linear(fmt, B):
    assert linear_path("cublas", fmt, B, *QKV, True) == "linear"


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("shape", [QKV, IN, W13, W2, HEAD, OUT])
@pytest.mark.parametrize("B", [1, 2, 3, 8, 9, 16])
def test_quantized_gemv_up_to_16(fmt, shape, B):
    for kept in (True, False):
        assert linear_path(fmt, fmt, B, *shape, kept) == "gemv"


def test_int8_above_16():
    # the lm_head (32768+ rows): W8A16 up to 128 rows, then the kept BF16 copy
    for B in (17, 24, 64, 128):
        assert linear_path("int8", "int8", B, *HEAD, True) == "w8a16"
    assert [linear_path("int8", "int8", B, *HEAD, True) for B in (129, 512)] == ["linear", "linear"]
    assert [linear_path("int8", "int8", B, *HEAD, False) for B in (17, 129, 4096)] == ["w8a16"] * 3
    # w1|w3-sized weights (8192+ rows): W8A16 from batch 17 up to 256 rows
    assert [linear_path("int8", "int8", B, *W13, True) for B in (17, 24, 25, 256, 257)] == \
        ["w8a16", "w8a16", "w8a16", "w8a16", "linear"]
    assert [linear_path("int8", "int8", B, *W13, False) for B in (17, 257, 1024)] == ["w8a16"] * 3
    # narrow, K = 2048: the GEMV up to 32 rows, W8A16 up to 256, then the kept BF16 copy
    for shape in (QKV, IN, OUT):
        assert [linear_path("int8", "int8", B, *shape, True) for B in (17, 32, 33, 256, 257)] == \
            ["gemv", "gemv", "w8a16", "w8a16", "linear"]
        assert [linear_path("int8", "int8", B, *shape, False) for B in (17, 32, 33, 300)] == \
            ["gemv", "gemv", "w8a16", "w8a16"]
    # w2 (K = 8192): the kept BF16 copy up to 24 rows, W8A16 up to 256, the BF16 copy beyond; W8A16 without one
    assert [linear_path("int8", "int8", B, *W2, True) for B in (17, 24, 25, 256, 257)] == \
        ["linear", "linear", "w8a16", "w8a16", "linear"]
    assert [linear_path("int8", "int8", B, *W2, False) for B in (17, 48, 49, 1024)] == ["w8a16"] * 4


def test_int4_above_16():
    # with a kept BF16 copy: the GEMV (16-row chunks) up to 32 rows for narrow weights, 24 for w1|w3-sized ones, 48
    # for the lm_head, never for w2; F.linear beyond
    for shape in (QKV, IN, OUT):
        assert [linear_path("int4", "int4", B, *shape, True) for B in (17, 32, 33, 1000)] == \
            ["gemv", "gemv", "linear", "linear"]
    assert [linear_path("int4", "int4", B, *W13, True) for B in (17, 24, 25)] == ["gemv", "gemv", "linear"]
    assert [linear_path("int4", "int4", B, *HEAD, True) for B in (17, 48, 49)] == ["gemv", "gemv", "linear"]
    assert [linear_path("int4", "int4", B, *W2, True) for B in (17, 64)] == ["linear", "linear"]
    for shape in (QKV, W13, W2, HEAD):
        for B in (17, 64, 1000):
            assert linear_path("int4", "int4", B, *shape, False) == "gemv"  # no INT4 GEMM: the GEMV in 16-row chunks


def test_int8_weights_in_int4_mode():
    """w4_keep_int8 kinds are stored in INT8 under mode "int4" and follow the INT8 rules."""
    assert linear_path("int4", "int8", 24, *HEAD, True) == "w8a16"
    assert linear_path("int4", "int8", 40, *QKV, True) == "w8a16"
    assert linear_path("int4", "int8", 300, *QKV, True) == "linear"


def test_bf16_weights():
    assert [linear_path("bf16", "bf16", B, *QKV, False) for B in (1, 8, 9, 16, 17)] == \
        ["gemv", "gemv", "gemv", "gemv", "linear"]
    assert [linear_path("bf16", "bf16", B, *W2, False) for B in (1, 8, 9, 16)] == ["gemv", "gemv", "linear", "linear"]


def test_bad_arguments():
    with pytest.raises(ValueError):
        linear_path("fp8", "int8", 1, *QKV, True)
    with pytest.raises(ValueError):
        linear_path("int8", "fp4", 1, *QKV, True)
