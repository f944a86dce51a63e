"""CPU oracle for the quantized matrix-multiply hot path (numpy front end over oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as what results are compared with. The product (liblfm2q.so and the lfm2opt package) never imports or
calls it.

bf16 arrays are numpy uint16 arrays holding the raw bf16 bit patterns. Every function cites the reference code it
restates (paths relative to the reference repository root); the arithmetic itself lives in oracle.c.
"""

import ctypes
import pathlib

import numpy as np

_LIB_PATH = pathlib.Path(__file__).resolve().with_name("liboracle.so")
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_SIGS = {
    "orc_f2bf": ([ctypes.c_float], ctypes.c_uint16),
    "orc_bf2f": ([ctypes.c_uint16], ctypes.c_float),
    "orc_f2bf_array": ([_P, _I64, _P], None),
    "orc_silu": ([ctypes.c_float], ctypes.c_float),
    "orc_gelu_tanh": ([ctypes.c_float], ctypes.c_float),
    "orc_f16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
    "orc_silu_mul": ([_P, _I64, _I64, _P], None),
    "orc_quant_rows": ([_P, _I64, _I64, _P, _P], None),
    "orc_quant_groups": ([_P, _I64, _I64, _P, _P], None),
    "orc_add_rmsnorm": ([_P, _P, _P, _I64, _I64, ctypes.c_float, _P], None),
    "orc_gemm_w8": ([_P, _P, _P, _P, _I64, _I64, _I64, _INT, _P], None),
    "orc_add_layernorm": ([_P, _P, _P, _P, _I64, _I64, ctypes.c_float, _P], None),
    "orc_gemm_i8_i32": ([_P, _P, _I64, _I64, _I64, _P], None),
    "orc_gemm_i8_epilogue": ([_P, _P, _P, _P, _I64, _I64, _INT, _P], None),
    "orc_gemm_i8_grouped": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _INT, _P], None),
    "orc_gemv": ([_P, _INT, _P, _P, _I64, _I64, _I64, _P], None),
    "orc_gemv_swiglu": ([_P, _INT, _P, _P, _I64, _I64, _I64, _P], None),
    "orc_gemv_residual": ([_P, _INT, _P, _P, _I64, _I64, _I64, _P], None),
    "orc_gemv_w4": ([_P, _P, _P, _I64, _I64, _I64, _I64, _P], None),
    "orc_gemv_w4z": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P], None),
}


def lib():
    """The compiled restatement (oracle/liboracle.so, built by `make -C oracle`)."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"{_LIB_PATH} is not built: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(_LIB_PATH))
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, res
        _lib = L
    return _lib


def _c(a, dtype):
    """C-contiguous array of `dtype` (no copy when it already is one)."""
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------------------------------------------ bf16
def f2bf(x):
    """fp32 -> bf16 bits, round to nearest even (torch .to(torch.bfloat16))."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f2bf_array(_p(x), x.size, _p(y))
    return y


def bf2f(h):
    """bf16 bits -> fp32 (exact)."""
    return (_c(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------------------------------------ quant
def quant_rows(x):
    """x bf16 [rows, K] -> (q int8 [rows, K], s fp32 [rows]); tests/test_int8_gemm.py:35-38 (ref_quant),
    kernels/int8_gemm.cu:391-432."""
    x = _c(x, np.uint16)
    rows, K = x.shape
    q = np.empty((rows, K), np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quant_rows(_p(x), rows, K, _p(q), _p(s))
    return q, s


def add_rmsnorm(h, y, w, eps):
    """-> (h_new, x): h_new = bf16(h + y) (h unchanged if y is None), x = bf16(w * bf16(h_new * rsqrt(mean(h_new^2) +
    eps))); bf16 as uint16 bits (kernels/lfm2_decode.cu:96-121, the input of add_rmsnorm_q)."""
    hn = _c(np.array(h, copy=True), np.uint16)
    rows, H = hn.shape
    x = np.empty_like(hn)
    lib().orc_add_rmsnorm(_p(hn), None if y is None else _p(_c(y, np.uint16)), _p(_c(w, np.uint16)), rows, H,
                          float(eps), _p(x))
    return hn, x


def add_layernorm(h, y, w, b, eps):
    """-> (h_new, x): h_new = bf16(h + y), x = bf16(LayerNorm(h_new) * w + b) (kernels/vision_ops.cu:29-80)."""
    hn = _c(np.array(h, copy=True), np.uint16)
    rows, D = hn.shape
    x = np.empty_like(hn)
    lib().orc_add_layernorm(_p(hn), None if y is None else _p(_c(y, np.uint16)), _p(_c(w, np.uint16)),
                            _p(_c(b, np.uint16)), rows, D, float(eps), _p(x))
    return hn, x


def quant_groups(x):
    """x bf16 [rows, K] -> (q int8 [rows, K], sT fp32 [K/64, rows]); tests/test_int8_gemm.py:64-69,
    kernels/int8_gemm.cu:435-474."""
    x = _c(x, np.uint16)
    rows, K = x.shape
    assert K % 64 == 0
    q = np.empty((rows, K), np.int8)
    sT = np.empty((K // 64, rows), np.float32)
    lib().orc_quant_groups(_p(x), rows, K, _p(q), _p(sT))
    return q, sT


# ------------------------------------------------------------------------------------------------ W8A8
def gemm_i8_i32(A, B):
    """Exact int32 C = A @ B^T for A int8 [M, K], B int8 [N, K] (the torch._int_mm analogue)."""
    A, B = _c(A, np.int8), _c(B, np.int8)
    (M, K), (N, K2) = A.shape, B.shape
    assert K == K2
    C = np.empty((M, N), np.int32)
    lib().orc_gemm_i8_i32(_p(A), _p(B), M, N, K, _p(C))
    return C


def gemm_i8_epilogue(C, sx, sw, bias=None, gelu=False):
    """bf16(gelu?(((float)C * sx[m]) * sw[n] + b[n])) -- kernels/int8_gemm.cu:93-115 (store_tile)."""
    C = _c(C, np.int32)
    M, N = C.shape
    sx, sw = _c(sx, np.float32), _c(sw, np.float32)
    b = None if bias is None else _c(bias, np.uint16)
    Y = np.empty((M, N), np.uint16)
    lib().orc_gemm_i8_epilogue(_p(C), _p(sx), _p(sw), _p(b), M, N, int(gelu), _p(Y))
    return Y


def gemm_i8(A, sx, B, sw, bias=None, gelu=False):
    """Per-token W8A8: gemm_i8_kernel<BM, 3, GELU, false, false>, kernels/int8_gemm.cu:125-297."""
    return gemm_i8_epilogue(gemm_i8_i32(A, B), sx, sw, bias, gelu)


def gemm_i8_grouped(A, sxT, B, sw, bias=None, gelu=False):
    """Grouped-64 W8A8 fold: kernels/int8_gemm.cu:202-230 then :93-115."""
    A, B = _c(A, np.int8), _c(B, np.int8)
    (M, K), (N, _) = A.shape, B.shape
    sxT, sw = _c(sxT, np.float32), _c(sw, np.float32)
    b = None if bias is None else _c(bias, np.uint16)
    Y = np.empty((M, N), np.uint16)
    lib().orc_gemm_i8_grouped(_p(A), _p(sxT), _p(B), _p(sw), _p(b), M, N, K, int(gelu), _p(Y))
    return Y


def gemm_w8(x, W, sw, bias=None, gelu=False):
    """W8A16: bf16 x [M, K] (uint16 bits) . int8 W [N, K]^T in fp64 -> fp32, * sw[n] + b[n], GELU, bf16
    (kernels/int8_gemm.cu:306-388, store_tile without activation scales)."""
    x, W, sw = _c(x, np.uint16), _c(W, np.int8), _c(sw, np.float32)
    (M, K), (N, _) = x.shape, W.shape
    b = None if bias is None else _c(bias, np.uint16)
    Y = np.empty((M, N), np.uint16)
    lib().orc_gemm_w8(_p(x), _p(W), _p(sw), _p(b), M, N, K, int(gelu), _p(Y))
    return Y


# ------------------------------------------------------------------------------------------------ GEMVs
def _wt(W):
    if W.dtype == np.int8:
        return _c(W, np.int8), 0
    assert W.dtype == np.uint16, "W: int8, or bf16 bits as uint16"
    return _c(W, np.uint16), 1


def gemv(W, scale, x):
    """y[b, n] = bf16((sum_k W[n, k] x[b, k]) * scale[n]); kernels/lfm2_decode.cu:576-661."""
    W, wt = _wt(W)
    x = _c(np.atleast_2d(x), np.uint16)
    N, K = W.shape
    B = x.shape[0]
    sc = None if scale is None else _c(scale, np.float32)
    y = np.empty((B, N), np.uint16)
    lib().orc_gemv(_p(W), wt, _p(sc), _p(x), B, N, K, _p(y))
    return y


def gemv_swiglu(W, scale, x):
    """W = w1|w3 [2S, K] -> y [B, S] = bf16(bf16(silu(g)) u); kernels/lfm2_decode.cu:724-805 (EPI 0)."""
    W, wt = _wt(W)
    x = _c(np.atleast_2d(x), np.uint16)
    S2, K = W.shape
    B = x.shape[0]
    sc = None if scale is None else _c(scale, np.float32)
    y = np.empty((B, S2 // 2), np.uint16)
    lib().orc_gemv_swiglu(_p(W), wt, _p(sc), _p(x), B, S2 // 2, K, _p(y))
    return y


def gemv_residual(W, scale, x, h):
    """Returns h_new = bf16(h + bf16(acc * s)); kernels/lfm2_decode.cu:108-113 rounding."""
    W, wt = _wt(W)
    x = _c(np.atleast_2d(x), np.uint16)
    N, K = W.shape
    B = x.shape[0]
    sc = None if scale is None else _c(scale, np.float32)
    hn = np.array(np.atleast_2d(h), np.uint16, copy=True, order="C")
    lib().orc_gemv_residual(_p(W), wt, _p(sc), _p(x), B, N, K, _p(hn))
    return hn


def silu_mul(g):
    """g bf16 [B, 2I] -> y bf16 [B, I]; kernels/lfm2_decode.cu:954-963."""
    g = _c(np.atleast_2d(g), np.uint16)
    B, I2 = g.shape
    y = np.empty((B, I2 // 2), np.uint16)
    lib().orc_silu_mul(_p(g), B, I2 // 2, _p(y))
    return y


def gemv_w4(Wp, S, x):
    """Reference INT4 format (uint8 [N, K/2] nibbles, q + 8; fp32 S [N, K/group]); kernels/lfm2_decode.cu:833-924."""
    Wp, S = _c(Wp, np.uint8), _c(S, np.float32)
    x = _c(np.atleast_2d(x), np.uint16)
    N, K2 = Wp.shape
    K = 2 * K2
    group = K // S.shape[1]
    B = x.shape[0]
    y = np.empty((B, N), np.uint16)
    lib().orc_gemv_w4(_p(Wp), _p(S), _p(x), B, N, K, group, _p(y))
    return y


def gemv_w4z(Wq, S, Z, x, group, swiglu=False):
    """GPTQ-style INT4 with zero points: Wq int32 [N, K/8], S fp16 [N, K/group] (as float16 or uint16 bits),
    Z int32 [N, ceil(G/8)]; w = s (q - z). swiglu: W = w1|w3 and y [B, N/2]."""
    Wq, Z = _c(Wq, np.int32), _c(Z, np.int32)
    S = _c(np.asarray(S).view(np.uint16) if np.asarray(S).dtype == np.float16 else S, np.uint16)
    x = _c(np.atleast_2d(x), np.uint16)
    N, K8 = Wq.shape
    K = 8 * K8
    B = x.shape[0]
    Nout = N // 2 if swiglu else N
    y = np.empty((B, Nout), np.uint16)
    lib().orc_gemv_w4z(_p(Wq), _p(S), _p(Z), _p(x), B, Nout, K, group, int(swiglu), _p(y))
    return y


# ------------------------------------------------------------------------------------------------ scalars
def silu_scalar(g):
    return lib().orc_silu(float(g))


def gelu_scalar(v):
    return lib().orc_gelu_tanh(float(v))


def f16_to_f32_scalar(h):
    return lib().orc_f16_to_f32(int(h))
