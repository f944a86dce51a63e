"""Extension entry points with the reference's Python surface, backed by the gfx950 library liblfm2q.so.

`ext()` stands in for the JIT-built decode extension and `int8_ext()` for the INT8 GEMM extension of
src/lfm2opt/kernels.py:16-32,66-68. The ops keep their names, argument order and meaning, destination-passing
style (every output is preallocated by the caller, ops return None) and launch on torch's current stream. Argument
errors raise RuntimeError with the reference's TORCH_CHECK wording (kernels/lfm2_decode.cpp:28-150) before any
launch. Ops outside the quantized-matmul path (attention, norms, convolutions) are not provided.
"""

import ctypes
import os

import torch

from . import _capi

# The per-stream GEMM workspace (the K split across workgroups): create it on a capture stream before capturing,
# release it when a stream is retired.
prepare_workspace = _capi.prepare_workspace
release_workspace = _capi.release_workspace

_EXT = None


def _check_bf16(t, name):
    if not (t.is_cuda and t.dtype == torch.bfloat16 and t.is_contiguous()):
        raise RuntimeError(f"{name} must be contiguous CUDA bf16")


def _check_t(t, dtype, name):
    if not (t.is_cuda and t.dtype == dtype and t.is_contiguous()):
        raise RuntimeError(f"{name} must be contiguous CUDA {dtype}")


def _same_device(*ts):
    dev = ts[0].device
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise RuntimeError("all tensors must be on the same device")


class DecodeOps:
    """Decode-path ops (reference: kernels/lfm2_decode.cpp)."""

    def __init__(self):
        _capi.lib()
        self.pdl = True
        self.gemv_impl = 1

    # ---- reference ops ------------------------------------------------------------------------------------
    def gemv(self, W, scale, x, y, rows=0):
        """y [B, N] = x [B, K] @ W^T, W [N, K] bf16 or int8 (then scale [N] fp32 is required); any B >= 1.
        Reference: gemv(), kernels/lfm2_decode.cpp:74-85. rows: output rows per wavefront for B == 1."""
        _check_bf16(x, "x")
        _check_bf16(y, "y")
        if not (W.is_cuda and W.is_contiguous() and W.dim() == 2):
            raise RuntimeError("W must be a contiguous CUDA matrix")
        int8 = W.dtype == torch.int8
        if not (int8 or W.dtype == torch.bfloat16):
            raise RuntimeError("W must be bf16 or int8")
        if int8 and (scale is None or scale.dtype != torch.float32):
            raise RuntimeError("int8 W needs fp32 scale")
        N, K = W.shape
        B = x.numel() // K if K else 0
        if not (B >= 1 and x.numel() == B * K and y.numel() == B * N):
            raise RuntimeError("x [B, K], y [B, N]")
        if scale is not None:
            _check_t(scale, torch.float32, "scale")
            if scale.numel() != N:
                raise RuntimeError("scale must have N elements")
        _same_device(W, x, y, scale)
        fn = "lfm2q_gemv_w8" if int8 else "lfm2q_gemv_bf16"
        _capi.call(fn, W.data_ptr(), _capi.ptr(scale), x.data_ptr(), y.data_ptr(), B, N, K, int(rows),
                   _capi.stream(x))

    def gemv_epi(self, epi, W, scale, x, y, state=None, cw=None, cbias=None):
        """epi 0: W = w1|w3 [2S, K] -> y [B, S] = silu(w1 x) * (w3 x), fused into the GEMV.
        Reference: gemv_epi(), kernels/lfm2_decode.cpp:130-150 (batch 1 there; any B >= 1 here). epi 1 (the LFM2
        short-conv step) is not a matmul epilogue and is not provided by this library."""
        if epi != 0:
            if epi == 1:
                raise RuntimeError("gemv_epi: epi 1 (short-conv step) is outside the quantized-matmul library")
            raise RuntimeError("epi 0 (swiglu) or 1 (shortconv)")
        W, scale, B, S, K, wtype = self._epi_args(W, scale, x, y, rows_per_out=2)
        _capi.call("lfm2q_gemv_swiglu", wtype, W.data_ptr(), _capi.ptr(scale), x.data_ptr(), y.data_ptr(), B, S, K,
                   _capi.stream(x))

    def gemv_w4(self, Wp, S, x, y, rows=0, epi=0):
        """INT4 weight-only GEMV in the reference format: Wp uint8 [R, K/2] (two int4 + 8 per byte, weight 2j in the
        low nibble of byte j), S fp32 [R, K/group]; y [B, N] = x [B, K] @ dequant(Wp)^T with R = N.
        Reference: gemv_w4(), kernels/lfm2_decode.cpp:86-98 (batch 1 there; any B >= 1 here). rows is accepted for
        the reference's signature and has no effect. epi (an addition): 0 plain, 1 SwiGLU over Wp = w1|w3
        (R = 2N, y [B, N]), 2 residual add in place into y."""
        _check_bf16(x, "x")
        _check_bf16(y, "y")
        if not (Wp.is_cuda and Wp.is_contiguous() and Wp.dtype == torch.uint8 and Wp.dim() == 2):
            raise RuntimeError("Wp: contiguous uint8 [N, K/2]")
        if not (S.is_cuda and S.is_contiguous() and S.dtype == torch.float32):
            raise RuntimeError("S: contiguous fp32 [N, K/128]")
        R, K = Wp.size(0), Wp.size(1) * 2
        group = self._w4_group(S, R, K)
        B, N = self._w4_shapes(x, y, R, K, epi)
        _same_device(Wp, S, x, y)
        _capi.call("lfm2q_gemv_w4", 0, Wp.data_ptr(), S.data_ptr(), None, x.data_ptr(), y.data_ptr(), B, N, K, group,
                   int(epi), _capi.stream(x))

    def gemv_w4z(self, qweight, scales, qzeros, x, y, epi=0):
        """INT4 weight-only GEMV in GPTQ-style storage (an addition): qweight int32 [R, K/8] (nibble i of word w =
        q for k = 8 w + i, q in [0, 15]), scales fp16 [R, K/group], qzeros int32 [R, ceil(K/group/8)] (nibble j of
        word w = zero point of group 8 w + j); w = s (q - z). epi as in gemv_w4."""
        _check_bf16(x, "x")
        _check_bf16(y, "y")
        if not (qweight.is_cuda and qweight.is_contiguous() and qweight.dtype == torch.int32 and qweight.dim() == 2):
            raise RuntimeError("qweight: contiguous int32 [N, K/8]")
        if not (scales.is_cuda and scales.is_contiguous() and scales.dtype == torch.float16):
            raise RuntimeError("scales: contiguous fp16 [N, K/group]")
        R, K = qweight.size(0), qweight.size(1) * 8
        group = self._w4_group(scales, R, K)
        G = K // group
        if not (qzeros.is_cuda and qzeros.is_contiguous() and qzeros.dtype == torch.int32
                and tuple(qzeros.shape) == (R, (G + 7) // 8)):
            raise RuntimeError("qzeros: contiguous int32 [N, ceil(K/group/8)]")
        B, N = self._w4_shapes(x, y, R, K, epi)
        _same_device(qweight, scales, qzeros, x, y)
        _capi.call("lfm2q_gemv_w4", 1, qweight.data_ptr(), scales.data_ptr(), qzeros.data_ptr(), x.data_ptr(),
                   y.data_ptr(), B, N, K, group, int(epi), _capi.stream(x))

    @staticmethod
    def _w4_group(S, R, K):
        if not (S.dim() == 2 and S.size(0) == R and S.size(1) >= 1 and K % S.size(1) == 0):
            raise RuntimeError("S must be [N, K / group]")
        group = K // S.size(1)
        if group % 32:
            raise RuntimeError("group size must be a multiple of 32")
        return group

    @staticmethod
    def _w4_shapes(x, y, R, K, epi):
        if epi not in (0, 1, 2):
            raise RuntimeError("epi 0 (none), 1 (swiglu) or 2 (residual)")
        N = R // 2 if epi == 1 else R
        B = x.numel() // K if K else 0
        if not ((epi != 1 or R % 2 == 0) and B >= 1 and x.numel() == B * K and y.numel() == B * N):
            raise RuntimeError("x [B, K], y [B, N]")
        return B, N

    def silu_mul(self, g, y):
        """y = silu(a) * b on g = [a | b]; reference: silu_mul(), kernels/lfm2_decode.cpp:100-103."""
        _check_bf16(g, "g")
        _check_bf16(y, "y")
        I2 = g.size(-1)
        B = g.numel() // I2
        if I2 % 2 or y.numel() != B * (I2 // 2):
            raise RuntimeError("g [B, 2I], y [B, I]")
        _same_device(g, y)
        _capi.call("lfm2q_silu_mul", g.data_ptr(), y.data_ptr(), B, I2 // 2, _capi.stream(g))

    def gemv_chain(self, ops):
        """A GemvChain over ops [(epi, W, scale, x, y), ...] (an addition): call it to run all of them in one launch."""
        return GemvChain(ops)

    def set_pdl(self, on):
        """Accepted for compatibility (kernels/lfm2_decode.cpp:165); HIP has no programmatic dependent launch,
        back-to-back kernels on one stream are ordered by the stream and captured into HIP graphs instead."""
        self.pdl = bool(on)

    def set_gemv_impl(self, impl):
        """Accepted for compatibility (kernels/lfm2_decode.cpp:166): there is one GEMV implementation per batch
        size class here, so the choice between shared-memory and direct activation loads has no effect."""
        if impl not in (0, 1):
            raise RuntimeError("GEMV implementation: 0 = x staged in shared memory, 1 = direct x loads")
        self.gemv_impl = int(impl)

    # ---- additions ----------------------------------------------------------------------------------------
    def gemv_rmsnorm(self, W, scale, h, norm_w, eps, y, epi=0):
        """The batch-1 GEMV of RMSNorm(h) (an addition): x = bf16(norm_w * bf16(h * rsqrt(mean(h^2) + eps))) is
        formed inside the GEMV, then y [1, N] = x @ W^T * scale (epi 0) or the SwiGLU of x over W = w1|w3 (epi 1, y
        [1, N] from W [2N, K]). Bit-identical to add_rmsnorm (no residual input) followed by gemv / gemv_epi(0), the
        pair the reference's decode step runs before each of these linears (src/lfm2opt/runtime.py:251-255,
        :276-285). h, norm_w bf16 [K]; W int8 (K in 1024 .. 8192, powers of two, fp32 scale) or bf16 (K in 512 ..
        4096, scale optional)."""
        _check_bf16(h, "h")
        _check_bf16(norm_w, "norm_w")
        _check_bf16(y, "y")
        if epi not in (0, 1):
            raise RuntimeError("gemv_rmsnorm: epi 0 (none) or 1 (swiglu)")
        if not (W.is_cuda and W.is_contiguous() and W.dim() == 2 and W.dtype in (torch.int8, torch.bfloat16)):
            raise RuntimeError("W must be a contiguous CUDA bf16 or int8 matrix")
        int8 = W.dtype == torch.int8
        R, K = W.shape
        N = R // 2 if epi == 1 else R
        if int8 and (scale is None or scale.dtype != torch.float32):
            raise RuntimeError("int8 W needs fp32 scale")
        if scale is not None:
            _check_t(scale, torch.float32, "scale")
            if scale.numel() != R:
                raise RuntimeError("scale must have one value per weight row")
        if (epi == 1 and R % 2) or h.numel() != K or norm_w.numel() != K or y.numel() != N:
            raise RuntimeError("gemv_rmsnorm: h [1, K], norm_w [K], y [1, N] (batch 1)")
        _same_device(W, h, norm_w, y, scale)
        _capi.call("lfm2q_gemv_rmsnorm", 0 if int8 else 1, int(epi), W.data_ptr(), _capi.ptr(scale), h.data_ptr(),
                   norm_w.data_ptr(), float(eps), y.data_ptr(), N, K, _capi.stream(h))

    def gemv_residual(self, W, scale, x, h):
        """h [B, N] += bf16(x @ W^T * scale) in place, rounded as the reference's residual add
        (kernels/lfm2_decode.cu:108-113): h = bf16(h + bf16(acc * s))."""
        W, scale, B, N, K, wtype = self._epi_args(W, scale, x, h, rows_per_out=1)
        _capi.call("lfm2q_gemv_residual", wtype, W.data_ptr(), _capi.ptr(scale), x.data_ptr(), h.data_ptr(), B, N,
                   K, _capi.stream(x))

    def _epi_args(self, W, scale, x, y, rows_per_out):
        _check_bf16(x, "x")
        _check_bf16(y, "y")
        if not (W.is_cuda and W.is_contiguous() and W.dim() == 2):
            raise RuntimeError("W must be a contiguous CUDA matrix")
        int8 = W.dtype == torch.int8
        if not (int8 or W.dtype == torch.bfloat16):
            raise RuntimeError("W must be bf16 or int8")
        if int8 and (scale is None or scale.dtype != torch.float32):
            raise RuntimeError("int8 W needs fp32 scale")
        Nw, K = W.shape
        Nout = Nw // rows_per_out
        B = x.numel() // K if K else 0
        if not (Nw == rows_per_out * Nout and B >= 1 and x.numel() == B * K and y.numel() == B * Nout):
            raise RuntimeError("x [B, K], y [B, N]" if rows_per_out == 1 else "x [B, K], W [2S, K], y [B, S]")
        if scale is not None:
            _check_t(scale, torch.float32, "scale")
            if scale.numel() != Nw:
                raise RuntimeError("scale must have one element per row of W")
        _same_device(W, x, y, scale)
        return W, scale, B, Nout, K, 0 if int8 else 1


class GemvChain:
    """A fixed sequence of batch-1 INT8 GEMVs run as one launch (lfm2q_gemv_chain): op j may read anything ops
    0 .. j-1 wrote; every output equals the separate gemv / gemv_epi(0) / gemv_residual call bit for bit.

    ops: (epi, W, scale, x, y) per GEMV -- epi 0 y = x W^T s, 1 SwiGLU over W = w1|w3 (y [1, S]), 2 y += x W^T s in
    place; W int8 [R, K] with K in {1024, 2048, 4096, 8192}, scale fp32 [R], x bf16 [1, K], y bf16 [1, N]. The
    tensors are kept alive and their addresses fixed in the table, so the chain is replayed on the same buffers
    (graph-capturable: one kernel launch, no allocation). The op table is copied to the device and a workspace
    allocated once, here."""

    def __init__(self, ops):
        if not ops:
            raise RuntimeError("gemv_chain: at least one op")
        lib = _capi.lib()
        self._keep, table = [], []
        dev = None
        for j, (epi, W, scale, x, y) in enumerate(ops):
            if epi not in (0, 1, 2):
                raise RuntimeError(f"gemv_chain: op {j}: epi 0 (none), 1 (swiglu) or 2 (residual)")
            _check_t(W, torch.int8, f"op {j}: W")
            _check_t(scale, torch.float32, f"op {j}: scale")
            _check_bf16(x, f"op {j}: x")
            _check_bf16(y, f"op {j}: y")
            R, K = W.shape
            N = R // 2 if epi == 1 else R
            if (epi == 1 and R % 2) or scale.numel() != R or x.numel() != K or y.numel() != N:
                raise RuntimeError(f"gemv_chain: op {j}: x [1, K], W [{'2N' if epi == 1 else 'N'}, K], y [1, N]")
            _same_device(W, scale, x, y)
            if dev is not None and W.device != dev:
                raise RuntimeError("all tensors must be on the same device")
            dev = W.device
            self._keep += [W, scale, x, y]
            table.append(_capi.GemvOp(W.data_ptr(), scale.data_ptr(), x.data_ptr(), y.data_ptr(), N, K, epi, 0))
        self.n = len(table)
        self.host = (_capi.GemvOp * self.n)(*table)
        self.dev = torch.frombuffer(bytearray(bytes(self.host)), dtype=torch.uint8).to(dev)
        self.ws_bytes = lib.lfm2q_gemv_chain_workspace_bytes()
        self.ws = torch.zeros(-(-self.ws_bytes // 4), dtype=torch.int32, device=dev)
        self.device = dev

    def __call__(self):
        with torch.cuda.device(self.device):
            _capi.call("lfm2q_gemv_chain", ctypes.addressof(self.host), self.dev.data_ptr(), self.n,
                       self.ws.data_ptr(), self.ws_bytes, torch.cuda.current_stream(self.device).cuda_stream)

    def wait_expired(self):
        """True if a dependency wait of the last launch on this chain ran out (its outputs are then undefined; the
        launches after it are not affected). Reads the workspace's launch count and error tag on the host
        (synchronizes)."""
        gen, tag = (int(v) for v in self.ws[:2].tolist())
        return gen != 0 and tag == gen


class Int8Ops:
    """INT8 prefill / vision ops (reference: kernels/int8_gemm.cpp): quantizers, fused producers, the W8A8 GEMM with
    per-token or grouped-64 activation scales, its INT8-output form gemm_i8_q, and the W8A16 gemm_w8."""

    def __init__(self):
        _capi.lib()

    def gemm_i8(self, xq, sx, w, sw, bias, y, gelu):
        """W8A8: y [M, N] = bf16(gelu?((xq . w^T) * sx[m] * sw[n] + bias[n])), exact int32 accumulation; with 2-D sx
        [K/64, M] (grouped-64 activation scales) the per-group sums fold into fp32 with their scales first.
        Reference: gemm_i8(), kernels/int8_gemm.cpp:39-50."""
        _check_t(xq, torch.int8, "xq")
        _check_t(sx, torch.float32, "sx")
        K = xq.size(-1)
        M = xq.numel() // K if K else 0
        grouped = sx.dim() == 2
        if not ((K % 64 == 0 and sx.size(0) == K // 64 and sx.size(1) == M) if grouped else sx.numel() == M):
            raise RuntimeError("sx shape")
        N = self._check_common(w, sw, bias, y, M, K)
        _same_device(xq, sx, w, sw, bias, y)
        if grouped:
            _capi.call("lfm2q_gemm_i8_grouped", xq.data_ptr(), sx.data_ptr(), w.data_ptr(), sw.data_ptr(),
                       _capi.ptr(bias), y.data_ptr(), M, N, K, int(bool(gelu)), _capi.stream(xq))
        else:  # per-token: with the stream's workspace (the K split for shapes with fewer tiles than CUs)
            ws = _capi.workspace(xq)
            _capi.call("lfm2q_gemm_i8_ex", xq.data_ptr(), sx.data_ptr(), w.data_ptr(), sw.data_ptr(),
                       _capi.ptr(bias), y.data_ptr(), M, N, K, int(bool(gelu)), ws.data_ptr(), ws.numel(),
                       _capi.stream(xq))

    def gemm_i8_bf16a(self, x, sx, w, sw, bias, y, gelu):
        """The per-token pair quant_rows(x) + gemm_i8 as one call on bf16 activations x [M, K]: sx [M] receives the
        scales quant_rows would write, the GEMM quantizes x inside (no int8 copy of x), and y is bit-identical to
        the pair's. Reference pair: src/lfm2opt/int8.py:45-51 (quantize_rows, then gemm_i8)."""
        _check_bf16(x, "x")
        _check_t(sx, torch.float32, "sx")
        K = x.size(-1)
        M = x.numel() // K if K else 0
        if sx.numel() != M:
            raise RuntimeError("sx shape")
        N = self._check_common(w, sw, bias, y, M, K)
        _same_device(x, sx, w, sw, bias, y)
        _capi.call("lfm2q_gemm_i8_bf16a", x.data_ptr(), sx.data_ptr(), w.data_ptr(), sw.data_ptr(), _capi.ptr(bias),
                   y.data_ptr(), M, N, K, int(bool(gelu)), _capi.stream(x))

    def gemm_i8_fq(self, x, xq, sx, w, sw, bias, y, gelu):
        """The per-token pair quant_rows(x) -> (xq, sx), then gemm_i8, behind one call with the stream's workspace;
        xq, sx and y are bit-identical to the pair's. By default the library runs the pair; with the tuning knob
        LFM2Q_GEMM_FQ = 1 the persistent GEMM's workgroups quantize x first and then run the tiles, in one launch.
        Reference pair: src/lfm2opt/int8.py:45-51 (quantize_rows, then gemm_i8)."""
        _check_bf16(x, "x")
        _check_t(xq, torch.int8, "xq")
        _check_t(sx, torch.float32, "sx")
        K = x.size(-1)
        M = x.numel() // K if K else 0
        if xq.numel() != M * K or xq.size(-1) != K:
            raise RuntimeError("xq shape")
        if sx.numel() != M:
            raise RuntimeError("sx shape")
        N = self._check_common(w, sw, bias, y, M, K)
        _same_device(x, xq, sx, w, sw, bias, y)
        ws = _capi.workspace(x)
        _capi.call("lfm2q_gemm_i8_fq", x.data_ptr(), xq.data_ptr(), sx.data_ptr(), w.data_ptr(), sw.data_ptr(),
                   _capi.ptr(bias), y.data_ptr(), M, N, K, int(bool(gelu)), ws.data_ptr(), ws.numel(),
                   _capi.stream(x))

    def gemm_i8_q(self, xq, sxT, w, sw, bias, yq, ysT, gelu):
        """Grouped W8A8 writing the next W8A8 GEMM's input: (yq [M, N], ysT [N/64, M]) = quant_groups(the bf16 output
        gemm_i8 would write), bit-identical to that pair of calls. Reference: gemm_i8_q(), kernels/int8_gemm.cpp:53-69
        (N % 128 there, N % 64 here)."""
        for t, dt, name in ((xq, torch.int8, "xq"), (sxT, torch.float32, "sxT"), (w, torch.int8, "w"),
                            (sw, torch.float32, "sw"), (yq, torch.int8, "yq"), (ysT, torch.float32, "ysT")):
            _check_t(t, dt, name)
        K = xq.size(-1)
        M = xq.numel() // K if K else 0
        N = w.size(0)
        if not (sxT.dim() == 2 and K % 64 == 0 and sxT.size(0) == K // 64 and sxT.size(1) == M):
            raise RuntimeError("sxT shape")
        if not (w.dim() == 2 and w.size(1) == K and N % 64 == 0 and sw.numel() == N):
            raise RuntimeError("w [N, K] with N % 64 == 0")
        if not (yq.numel() == M * N and ysT.dim() == 2 and ysT.size(0) == N // 64 and ysT.size(1) == M):
            raise RuntimeError("yq / ysT shape")
        if bias is not None:
            _check_bf16(bias, "bias")
            if bias.numel() != N:
                raise RuntimeError("bias shape")
        _same_device(xq, sxT, w, sw, bias, yq, ysT)
        _capi.call("lfm2q_gemm_i8_q", xq.data_ptr(), sxT.data_ptr(), w.data_ptr(), sw.data_ptr(), _capi.ptr(bias),
                   yq.data_ptr(), ysT.data_ptr(), M, N, K, int(bool(gelu)), _capi.stream(xq))

    def gemm_w8(self, x, w, sw, bias, y, gelu):
        """W8A16: y [M, N] = bf16(gelu?((x . w^T) * sw[n] + bias[n])), bf16 x, int8 w, fp32 accumulation.
        Reference: gemm_w8(), kernels/int8_gemm.cpp:72-79."""
        _check_bf16(x, "x")
        K = x.size(-1)
        M = x.numel() // K if K else 0
        N = self._check_common(w, sw, bias, y, M, K)
        _same_device(x, w, sw, bias, y)
        ws = _capi.workspace(x)  # the K split across workgroups for shapes with few tiles
        _capi.call("lfm2q_gemm_w8_ex", x.data_ptr(), w.data_ptr(), sw.data_ptr(), _capi.ptr(bias), y.data_ptr(), M, N,
                   K, int(bool(gelu)), ws.data_ptr(), ws.numel(), _capi.stream(x))

    def gemm_i8_i32(self, xq, w, c):
        """The exact int32 accumulators c [M, N] = xq [M, K] . w [N, K]^T (the torch._int_mm analogue)."""
        _check_t(xq, torch.int8, "xq")
        _check_t(w, torch.int8, "w")
        _check_t(c, torch.int32, "c")
        K = xq.size(-1)
        M = xq.numel() // K if K else 0
        if not (w.dim() == 2 and w.size(1) == K):
            raise RuntimeError("w must be [N, K]")
        N = w.size(0)
        if c.numel() != M * N:
            raise RuntimeError("c shape")
        if K % 16:
            raise RuntimeError("need K % 16 == 0")
        _same_device(xq, w, c)
        _capi.call("lfm2q_gemm_i8_i32", xq.data_ptr(), w.data_ptr(), c.data_ptr(), M, N, K, _capi.stream(xq))

    def quant_rows(self, x, q, s):
        """Symmetric quantization: s = max|x| / 127, q = round(x / s), per row (1-D s [rows]) or per row and group of
        64 columns (2-D s [K/64, rows], transposed as gemm_i8 reads it). Reference: quant_rows(),
        kernels/int8_gemm.cpp:83-96 (K % 128 and, per row, K <= 2048 there; K % 8, grouped K % 64, any K here)."""
        _check_bf16(x, "x")
        _check_t(q, torch.int8, "q")
        _check_t(s, torch.float32, "s")
        K = x.size(-1)
        rows = x.numel() // K if K else 0
        if s.dim() == 2:
            if not (K % 64 == 0 and K > 0 and s.size(0) == K // 64 and s.size(1) == rows and q.numel() == x.numel()):
                raise RuntimeError("grouped shapes")
            _same_device(x, q, s)
            _capi.call("lfm2q_quant_groups", x.data_ptr(), q.data_ptr(), s.data_ptr(), rows, K, _capi.stream(x))
            return
        if K % 8 or K == 0:
            raise RuntimeError("K must be a multiple of 8")
        if q.numel() != x.numel() or s.numel() != rows:
            raise RuntimeError("q / s shape")
        _same_device(x, q, s)
        _capi.call("lfm2q_quant_rows", x.data_ptr(), q.data_ptr(), s.data_ptr(), rows, K, _capi.stream(x))

    # ---- fused producers (kernels/int8_gemm.cpp:99-141). x (an addition): also write the bf16 row that was
    # quantized; q / s are then exactly quant_rows(x, ...) of it.
    @staticmethod
    def _check_qs(q, s, rows, L):
        """kernels/int8_gemm.cpp:99-105: per-row (1-D s) or grouped (2-D s [L/64, rows])."""
        _check_t(q, torch.int8, "q")
        _check_t(s, torch.float32, "s")
        grouped = s.dim() == 2
        if q.numel() != rows * L:
            raise RuntimeError("q shape")
        if not (s.size(0) == L // 64 and s.size(1) == rows and L % 64 == 0 if grouped else s.numel() == rows):
            raise RuntimeError("s shape")
        return int(grouped)

    def add_layernorm_q(self, h, y, w, b, q, s, eps, x=None):
        """vision: h += y (optional, in place, bf16-rounded); (q, s) = quant(LayerNorm(h) * w + b).
        Reference: add_layernorm_q(), kernels/int8_gemm.cpp:108-119 (D % 128, D <= 2048 there; D % 8, D <= 8192)."""
        _check_bf16(h, "h")
        _check_bf16(w, "w")
        _check_bf16(b, "b")
        if y is not None:
            _check_bf16(y, "y")
            if y.numel() != h.numel():
                raise RuntimeError("y shape")
        D = h.size(-1)
        rows = h.numel() // D if D else 0
        if not (D % 8 == 0 and 0 < D <= 8192 and w.numel() == D and b.numel() == D):
            raise RuntimeError("D must be a multiple of 8, <= 8192")
        grouped = self._check_qs(q, s, rows, D)
        if x is not None:
            _check_bf16(x, "x")
            if x.numel() != h.numel():
                raise RuntimeError("x shape")
        _same_device(h, y, w, b, q, s, x)
        _capi.call("lfm2q_add_layernorm_q", h.data_ptr(), _capi.ptr(y), w.data_ptr(), b.data_ptr(), q.data_ptr(),
                   s.data_ptr(), _capi.ptr(x), rows, D, float(eps), grouped, _capi.stream(h))

    def add_rmsnorm_q(self, h, y, w, q, s, eps, x=None):
        """LM prefill: h += y (optional, in place, bf16-rounded); (q, s) = quant(bf16(w * bf16(rmsnorm(h)))).
        Reference: add_rmsnorm_q(), kernels/int8_gemm.cpp:122-132 (H <= 8192 here)."""
        _check_bf16(h, "h")
        _check_bf16(w, "w")
        if y is not None:
            _check_bf16(y, "y")
            if y.numel() != h.numel():
                raise RuntimeError("y shape")
        H = h.size(-1)
        rows = h.numel() // H if H else 0
        if not (w.numel() == H and H % 8 == 0 and 0 < H <= 8192):
            raise RuntimeError("w shape")
        grouped = self._check_qs(q, s, rows, H)
        if x is not None:
            _check_bf16(x, "x")
            if x.numel() != h.numel():
                raise RuntimeError("x shape")
        _same_device(h, y, w, q, s, x)
        _capi.call("lfm2q_add_rmsnorm_q", h.data_ptr(), _capi.ptr(y), w.data_ptr(), q.data_ptr(), s.data_ptr(),
                   _capi.ptr(x), rows, H, float(eps), grouped, _capi.stream(h))

    def silu_mul_q(self, g, q, s, x=None):
        """LM prefill: g [rows, 2I] = w1 | w3 outputs -> (q, s) = quant(bf16(bf16(silu(g1)) * g3)).
        Reference: silu_mul_q(), kernels/int8_gemm.cpp:135-141 (I % 64, I <= 20000 there; I % 8, I <= 8192)."""
        _check_bf16(g, "g")
        I = g.size(-1) // 2
        rows = g.numel() // (2 * I) if I else 0
        if not (I % 8 == 0 and 0 < I <= 8192 and g.size(-1) == 2 * I):
            raise RuntimeError("I shape")
        grouped = self._check_qs(q, s, rows, I)
        if x is not None:
            _check_bf16(x, "x")
            if x.numel() != rows * I:
                raise RuntimeError("x shape")
        _same_device(g, q, s, x)
        _capi.call("lfm2q_silu_mul_q", g.data_ptr(), q.data_ptr(), s.data_ptr(), _capi.ptr(x), rows, I, grouped,
                   _capi.stream(g))

    @staticmethod
    def _check_common(w, sw, bias, y, M, K):
        """kernels/int8_gemm.cpp:22-36 (N % 8 is not required here)."""
        _check_t(w, torch.int8, "w")
        _check_t(sw, torch.float32, "sw")
        _check_bf16(y, "y")
        if not (w.dim() == 2 and w.size(1) == K):
            raise RuntimeError("w must be [N, K]")
        N = w.size(0)
        if K % 16:
            raise RuntimeError("need K % 16 == 0")
        if not (sw.numel() == N and y.numel() == M * N):
            raise RuntimeError("sw / y shape")
        if bias is not None:
            _check_bf16(bias, "bias")
            if bias.numel() != N:
                raise RuntimeError("bias shape")
        return N


_INT8 = None


def int8_ext():
    """INT8 GEMM ops for prefill and the vision encoder (reference: src/lfm2opt/kernels.py:66-68)."""
    global _INT8
    if _INT8 is None:
        _INT8 = Int8Ops()
    return _INT8


def ext():
    """The decode-op extension (reference: src/lfm2opt/kernels.py:16-32). LFM2_PDL is read like the reference
    does; it has no effect on HIP."""
    global _EXT
    if _EXT is None:
        _EXT = DecodeOps()
        _EXT.set_pdl(os.environ.get("LFM2_PDL", "1") != "0")
    return _EXT
