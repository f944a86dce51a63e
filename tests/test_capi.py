"""The C ABI without a GPU: liblfm2q.so loads, exports every function include/lfm2q.h declares, the ctypes table
matches the header, and argument errors come back as status codes (no kernel is launched for them)."""

import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "lfm2q.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(lfm2q_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from lfm2opt import _capi

    return _capi.lib()


def test_header_declares_entry_points():
    names = declared()
    assert "lfm2q_gemv_w8" in names and "lfm2q_last_error" in names


def test_library_exports_every_declared_symbol(L):
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    from lfm2opt import _capi

    assert sorted(_capi.SIGNATURES) == sorted(set(declared()) - {"lfm2q_last_error", "lfm2q_version"})


def test_calibration_library_exports_its_entry_point():
    """bench.py's MFMA-rate calibration (lib/liblfm2q_calib.so) is built beside the product library."""
    calib = ctypes.CDLL(str(ROOT / "lfm2.5-vl-optimization_amd" / "lib" / "liblfm2q_calib.so"))
    assert hasattr(calib, "lfm2q_calib_mfma_i8")


def test_version(L):
    assert L.lfm2q_version().decode().startswith("lfm2q")


def test_status_codes_without_launch(L):
    """Shape and pointer checks run on the host and return before any HIP call that launches work."""
    from lfm2opt import _capi

    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its argument check first
    assert _capi.lib().lfm2q_gemv_w8(None, None, None, None, 1, 64, 512, 0, None) == 1  # null pointers
    assert "null pointer" in L.lfm2q_last_error().decode()
    assert L.lfm2q_gemv_w8(fake, None, fake, fake, 1, 64, 512, 0, None) == 1  # int8 without scale
    assert L.lfm2q_gemv_w8(fake, fake, fake, fake, 1, 64, 96, 0, None) == 2  # K % 64
    assert "multiple of 64" in L.lfm2q_last_error().decode()
    assert L.lfm2q_gemv_w8(fake, fake, fake, fake, 0, 64, 512, 0, None) == 2  # B = 0
    assert L.lfm2q_gemv_w8(ctypes.c_void_p(0x1001), fake, fake, fake, 1, 64, 512, 0, None) == 3  # misaligned
    assert L.lfm2q_gemv_swiglu(2, fake, fake, fake, fake, 1, 64, 512, None) == 1  # bad wtype
    assert L.lfm2q_silu_mul(None, fake, 1, 8, None) == 1
    # the no-allocation chain: its op table (and so its scratch flags) hold at most 128 ops
    table = (_capi.GemvOp * 1)()
    assert L.lfm2q_gemv_chain_noalloc(None, fake, 1, None, None) == 1
    assert L.lfm2q_gemv_chain_noalloc(ctypes.addressof(table), fake, 129, None, None) == 2
    assert "at most 128" in L.lfm2q_last_error().decode()
    assert L.lfm2q_gemv_chain_noalloc(ctypes.addressof(table), fake, 0, None, None) == 2
    assert L.lfm2q_gemv_chain_noalloc(ctypes.addressof(table), ctypes.c_void_p(0x1008), 1, None, None) == 3
    # the W8A8 GEMM on bf16 activations: pointers, K % 16, alignment
    assert L.lfm2q_gemm_i8_bf16a(None, fake, fake, fake, None, fake, 4, 8, 64, 0, None) == 1
    assert L.lfm2q_gemm_i8_bf16a(fake, fake, fake, fake, None, fake, 4, 8, 72, 0, None) == 2
    assert "K % 16 == 0" in L.lfm2q_last_error().decode()
    assert L.lfm2q_gemm_i8_bf16a(fake, fake, fake, fake, None, fake, 0, 8, 64, 0, None) == 2
    assert L.lfm2q_gemm_i8_bf16a(ctypes.c_void_p(0x1008), fake, fake, fake, None, fake, 4, 8, 64, 0, None) == 3
    # the workspace forms: the plain entry point's checks, then a 256-byte aligned workspace of at least 64 KiB
    assert L.lfm2q_gemm_i8_ex(fake, fake, fake, fake, None, fake, 4, 8, 72, 0, None, 0, None) == 2
    assert L.lfm2q_gemm_i8_ex(fake, fake, fake, fake, None, fake, 4, 8, 64, 0, ctypes.c_void_p(0x1108), 1 << 20,
                              None) == 1
    assert "256-byte aligned" in L.lfm2q_last_error().decode()
    assert L.lfm2q_gemm_i8_ex(fake, fake, fake, fake, None, fake, 4, 8, 64, 0, fake, 4096, None) == 1
    assert L.lfm2q_gemm_w8_ex(fake, fake, fake, None, fake, 4, 8, 64, 0, ctypes.c_void_p(0x1108), 1 << 20, None) == 1
    assert L.lfm2q_gemm_w8_ex(None, fake, fake, None, fake, 4, 8, 64, 0, None, 0, None) == 1
    assert L.lfm2q_gemm_workspace_bytes() == 4 * 16384 + (64 << 20) + (256 << 10)
    ws = ctypes.c_void_p(0x100000)
    full = L.lfm2q_gemm_workspace_bytes()
    assert L.lfm2q_gemm_i8_fq(fake, fake, fake, fake, fake, None, fake, 4, 8, 64, 0, None, full, None) == 1
    assert "null pointer" in L.lfm2q_last_error().decode()
    assert L.lfm2q_gemm_i8_fq(fake, fake, fake, fake, fake, None, fake, 4, 8, 72, 0, ws, full, None) == 2
    assert L.lfm2q_gemm_i8_fq(fake, fake, fake, fake, fake, None, fake, 4, 8, 64, 0, ws, 64 << 20, None) == 1
    assert "at least" in L.lfm2q_last_error().decode()
    assert L.lfm2q_gemm_i8_fq(fake, fake, fake, fake, fake, None, fake, 4, 8, 64, 0, ctypes.c_void_p(0x100010), full,
                              None) == 1
    assert "256-byte aligned" in L.lfm2q_last_error().decode()


def test_python_checks_match_reference_wording():
    """The torch-facing layer raises RuntimeError with the reference's TORCH_CHECK text before reaching the C ABI
    (kernels/lfm2_decode.cpp:28-85); CPU tensors are rejected as non-CUDA."""
    import torch
    from lfm2opt.kernels import ext

    E = ext()
    W = torch.zeros(64, 512, dtype=torch.int8)
    x = torch.zeros(1, 512, dtype=torch.bfloat16)
    y = torch.zeros(1, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="must be contiguous CUDA bf16"):
        E.gemv(W, torch.ones(64), x, y)
    with pytest.raises(RuntimeError, match="GEMV implementation"):
        E.set_gemv_impl(3)
    E.set_pdl(False)
    E.set_gemv_impl(0)


def test_tuning_knobs_set_get_reset():
    """lfm2q_set_tuning / lfm2q_get_tuning: 1-4 integers per knob, NULL or "" back to automatic, unknown names and
    malformed values rejected with LFM2Q_ERR_ARG and a message (no GPU call involved)."""
    from lfm2opt import _capi

    _capi.set_tuning("LFM2Q_GEMV_MFMA", "1,2,8,2")
    assert _capi.get_tuning("LFM2Q_GEMV_MFMA") == (1, 2, 8, 2)
    _capi.set_tuning("LFM2Q_GEMM_RING", 644)
    assert _capi.get_tuning("LFM2Q_GEMM_RING") == (644,)
    _capi.set_tuning("LFM2Q_GEMV_WPC", "-3")
    assert _capi.get_tuning("LFM2Q_GEMV_WPC") == (-3,)
    for name in ("LFM2Q_GEMV_MFMA", "LFM2Q_GEMM_RING", "LFM2Q_GEMV_WPC"):
        _capi.set_tuning(name, None)
        assert _capi.get_tuning(name) == ()
    _capi.set_tuning("LFM2Q_GEMM_BM", "")
    assert _capi.get_tuning("LFM2Q_GEMM_BM") == ()
    for bad in ("1,2,3,4,5", "x", "1,", "1,,2", "99999", "3 4"):
        with pytest.raises(RuntimeError, match="expected 1 to 4 comma-separated integers"):
            _capi.set_tuning("LFM2Q_GEMV_MFMA", bad)
        assert _capi.get_tuning("LFM2Q_GEMV_MFMA") == ()  # a rejected value leaves the knob as it was
    with pytest.raises(RuntimeError, match="unknown knob"):
        _capi.set_tuning("LFM2Q_NO_SUCH_KNOB", "1")


def test_every_documented_knob_exists():
    """The header lists exactly the knobs the library defines (status.cpp's name table), and each is accepted by
    lfm2q_get_tuning."""
    from lfm2opt import _capi

    text = HEADER.read_text()
    listed = re.search(r"Knob names:\s*(.*?)\.\n", text, flags=re.S).group(1)
    names = []
    for prefix, body in re.findall(r"(LFM2Q_[A-Z0-9]+?)_\{([^}]*)\}", listed):
        names += [f"{prefix}_{n.strip()}" for n in body.split(",")]
    src = (HEADER.parent.parent / "lfm2.5-vl-optimization_amd" / "csrc" / "status.cpp").read_text()
    table = re.search(r"kKnobNames\[KNOB_COUNT\] = \{(.*?)\};", src, flags=re.S).group(1)
    assert sorted(names) == sorted(re.findall(r'"(LFM2Q_\w+)"', table))
    for n in names:
        _capi.get_tuning(n)
