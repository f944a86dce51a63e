"""INT8 linear layers of LM prefill and the vision encoder, on liblfm2q's gfx950 GEMMs.

Drop-in for the reference's src/lfm2opt/int8.py: the module exposes the same names with the same signatures and
environment switches, built on this package's Int8Ops (kernels.int8_ext()) and its C ABI.

Two ways to run a layer with INT8 weights (one fp32 scale per output row, quant.quantize_int8):
  W8A8   the bf16 activations are quantized to int8 first -- one scale per token, or per token and 64-column
         group -- then multiplied on the int8 matrix cores with exact int32 sums; the epilogue applies both scales
         (+ bias, + GELU) and writes bf16, or, with quant_out, the next W8A8 layer's int8 input.
  W8A16  bf16 activations against the int8 weights on the bf16 matrix cores (gemm_w8), fp32 sums.

Environment (read at each call, as the reference does):
  LFM2_INT8_GROUP        64 (default): activation scales per token and group of 64 input channels; 0: per token.
  LFM2_INT8_GROUP_KINDS  comma-separated layer kinds that use the groups; the others run per token.
  LFM2_INT8_A16          comma-separated layer kinds that keep bf16 activations (W8A16); a16_kinds() reads it.
Layers with more than 2048 input channels always use the groups.
"""

import os

import torch

from .kernels import int8_ext
from .quant import quantize_int8

GROUP_COLS = 64  # input channels per activation scale in grouped mode (one 64-byte K stage of the GEMM)
WIDE_K = 2048    # wider inputs always take grouped activation scales


class GroupSettingError(AssertionError, ValueError):
    """An LFM2_INT8_GROUP value other than 0 or 64. Catchable as AssertionError, like the reference's check, and as
    ValueError."""


def _kinds_from_env(var):
    """The set of layer kinds listed (comma-separated) in environment variable `var`."""
    return {k.strip() for k in os.environ.get(var, "").split(",") if k.strip()}


def a16_kinds():
    """Layer kinds whose activations stay bf16 (W8A16), from LFM2_INT8_A16 (reference: src/lfm2opt/int8.py:22-24)."""
    return _kinds_from_env("LFM2_INT8_A16")


def act_group(kind=None, K=0):
    """Activation-scale granularity of a W8A8 layer of kind `kind` with K input channels: 64 (a scale per token and
    64-channel group) or 0 (a scale per token). Reference: src/lfm2opt/int8.py:27-36."""
    setting = os.environ.get("LFM2_INT8_GROUP", str(GROUP_COLS))
    try:
        group = int(setting)
    except ValueError:
        group = None
    if group not in (0, GROUP_COLS):
        raise GroupSettingError(f"LFM2_INT8_GROUP must be 0 (per token) or {GROUP_COLS} (per 64-channel group), "
                                f"got {setting!r}")
    if K > WIDE_K:
        return GROUP_COLS
    only = _kinds_from_env("LFM2_INT8_GROUP_KINDS")
    return group if not only or kind in only else 0


def _scale_shape(rows, K, group):
    """Activation scales: [rows] per token, [K / 64, rows] per token and group (the transposed layout the GEMM
    reads)."""
    return (K // GROUP_COLS, rows) if group else (rows,)


def qbuf(rows, K, group, device):
    """Uninitialised (int8 [rows, K], fp32 scales) for a producer that writes a W8A8 layer's input (reference:
    src/lfm2opt/int8.py:39-42)."""
    q = torch.empty((rows, K), dtype=torch.int8, device=device)
    return q, torch.empty(_scale_shape(rows, K, group), dtype=torch.float32, device=device)


def quantize_rows(x2, group=0):
    """Symmetric int8 quantization of bf16 [M, K]: (q int8 [M, K], scales), one scale per row (group 0) or per row
    and 64-column group (group 64, scales [K / 64, M]). Reference: src/lfm2opt/int8.py:45-51."""
    rows, K = x2.shape
    q, s = qbuf(rows, K, group, x2.device)
    int8_ext().quant_rows(x2, q, s)
    return q, s


class Int8Linear:
    """y = x W^T (+ bias) (GELU) with INT8 weights, reference: src/lfm2opt/int8.py:54-91.

    Built from a bf16 weight [N, K] (quantized per output row here, after appending pad_n zero rows -- and pad_n
    zero bias entries -- and pad_k zero input columns) or from an already quantized pair (q int8 [N, K], scale fp32
    [N]). a8 selects W8A8 (else W8A16); kind names the layer for the LFM2_INT8_GROUP_KINDS rule."""

    def __init__(self, weight=None, bias=None, a8=True, q=None, scale=None, pad_n=0, pad_k=0, kind=None):
        if q is None:
            if weight is None:
                raise ValueError("Int8Linear needs a bf16 weight or a quantized (q, scale) pair")
            if pad_n or pad_k:
                weight = torch.nn.functional.pad(weight, (0, pad_k, 0, pad_n))
                if bias is not None and pad_n:
                    bias = torch.cat([bias, bias.new_zeros(pad_n)])
            q, scale = quantize_int8(weight)
        elif scale is None:
            raise ValueError("a quantized Int8Linear weight needs its per-row scale")
        self.q, self.s = q, scale
        self.bias = bias
        self.a8 = a8
        self.N, self.K = q.shape
        self.group = act_group(kind, self.K) if a8 else 0
        self.ext = int8_ext()

    # ---- the three GEMM forms ------------------------------------------------------------------------------------
    def _gemm_bf16_out(self, xq, sx, rows, gelu):
        y = torch.empty((rows, self.N), dtype=torch.bfloat16, device=xq.device)
        self.ext.gemm_i8(xq, sx, self.q, self.s, self.bias, y, gelu)
        return y

    def _gemm_int8_out(self, xq, sx, rows, gelu):
        """The next layer's grouped W8A8 input, quantized in this GEMM's epilogue (needs N % 64 == 0)."""
        if self.N % GROUP_COLS:
            raise RuntimeError(f"quant_out needs N % {GROUP_COLS} == 0 (N = {self.N})")
        yq, ys = qbuf(rows, self.N, GROUP_COLS, xq.device)
        self.ext.gemm_i8_q(xq, sx, self.q, self.s, self.bias, yq, ys, gelu)
        return yq, ys

    def _gemm_w8a16(self, x2, gelu):
        y = torch.empty((x2.shape[0], self.N), dtype=torch.bfloat16, device=x2.device)
        self.ext.gemm_w8(x2, self.q, self.s, self.bias, y, gelu)
        return y

    def __call__(self, x, gelu=False, quant_out=False):
        """x: bf16 [..., K], or (int8 [..., K], scales) already quantized by a fused producer. Returns bf16
        [..., N]; with quant_out, the next W8A8 layer's input (int8 [M, N], scales [N / 64, M]) instead, which needs
        grouped input scales (a bf16 x is quantized per 64-channel group for it)."""
        if isinstance(x, tuple):
            xq, sx = x
            lead = xq.shape[:-1]
            rows = xq.numel() // self.K
        else:
            lead = x.shape[:-1]
            x2 = x.reshape(-1, self.K).contiguous()
            rows = x2.shape[0]
            if not (self.a8 or quant_out):
                return self._gemm_w8a16(x2, gelu).view(*lead, self.N)
            xq, sx = quantize_rows(x2, GROUP_COLS if quant_out else self.group)
        if quant_out:
            return self._gemm_int8_out(xq, sx, rows, gelu)
        return self._gemm_bf16_out(xq, sx, rows, gelu).view(*lead, self.N)
