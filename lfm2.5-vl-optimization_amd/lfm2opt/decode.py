"""Decode-step linear layers by weight key, and the per-call choice between the GEMV kernels and a matrix-core GEMM.

Reference: StaticDecoder in src/lfm2opt/runtime.py -- load-time weight set-up :159-198 (quantization :173-186, kept
BF16 copies :175, W8A16 layers :194, drop_bf16 :196-215), _epi_ok :218-221, _linear :223-244, and the call sites that
fuse SwiGLU into the w1|w3 GEMV (:278-282).

Modes (the reference's `gemv` argument, runtime.py:63):
  "cublas"        every linear through torch.nn.functional.linear on the BF16 weight (hipBLASLt on ROCm);
  "bf16"          the BF16-weight GEMV;
  "int8", "int4"  weight-only quantized at construction (runtime.py:176-186): INT8 per-row scales; INT4 in groups of
                  w4_group, except the kinds in w4_keep_int8 (INT8) and the keys in w4_pre (pre-quantized, e.g. GPTQ
                  or AWQ output).

Dispatch (linear_path), from timings on MI355X at the LFM2 decode shapes (qkv 3072 x 2048, in_proj 6144 x 2048,
w1|w3 16384 x 2048, w2 2048 x 8192, lm_head 65536 x 2048):
  INT8 and INT4 weights, batch <= 16: the GEMV (e.g. INT8 w1|w3 9.8 us at batch 16 against 18 us for W8A16 and for
               BF16 F.linear); its fused SwiGLU and residual epilogues run at every batch size, where the reference
               fuses at batch 1 only (_epi_ok);
  INT8, batch > 16: W8A16, whose K split across workgroups keeps every CU busy from 17 rows on (w1|w3 12.3 us at
               17 rows against 13.5 for the GEMV, lm_head 33 against 37), except: narrow weights with K = 2048 keep
               the GEMV up to 32 rows (qkv 7.2 us against 10.9); w2 (K = 8192) takes the kept BF16 copy up to 24
               rows (13.9 us against 15.0); and with a kept BF16 copy F.linear takes over above 256 rows (128 for the
               lm_head, 32768+ rows: 77 us against 88 at 192 rows), where W8A16's per-tile weight conversion costs
               more than hipBLASLt's BF16 GEMM;
  INT4, batch > 16: the GEMV in 16-row chunks (no INT4 GEMM) while it beats F.linear on the kept BF16 copy -- up to
               32 rows for narrow weights with K = 2048 (qkv 10.0 us against 11.5 at 32 rows), 24 for w1|w3-sized
               ones (16.9 against 17.4), 48 for the lm_head (67 against 71) and never for w2 (15.9 against 13.8 at
               17 rows) -- then F.linear; without a BF16 copy always the GEMV;
  BF16 weights: the GEMV up to batch 8, and up to 16 for K < 8192 (qkv 6.6 us against 11.3 us for F.linear at
               batch 16; w2 18.5 against 13.1), F.linear beyond.
The reference's thresholds were measured on other GPUs (BF16 GEMV up to batch 4, INT8 up to 8, INT4 at batch 1).

AWQ: a pre-quantized INT4 entry may carry inv_s [K]; the GEMV then runs on x * inv_s (runtime.py:239-240). The
BF16 copy is the unscaled original weight, so F.linear takes x as it is.
"""

import os

import torch
import torch.nn.functional as F

from .int8 import Int8Linear
from .kernels import ext
from .quant import GROUP, quantize_int4, quantize_int8

MODES = ("cublas", "bf16", "int8", "int4")
GEMV_MAX_BATCH = 16      # quantized weights: the GEMV beat F.linear and W8A16 at every LFM2 shape up to this batch
BF16_GEMV_MAX_BATCH = 8  # BF16 weights (16 when K < 8192)
W8A16_MIN_ROWS = 8192    # INT8 weights with this many output rows (or K >= 8192) leave the GEMV above batch 16
GEMV_MAX_BATCH_NARROW = 32  # ... the others above batch 32
W8A16_MAX_BATCH = 256    # above this many rows a kept BF16 copy (F.linear) beats W8A16 ...
HEAD_ROWS = 32768        # ... and above 128 rows for weights with this many output rows


def linear_path(mode, fmt, B, N, K, has_bf16):
    """Which implementation computes a [B, K] x [N, K]^T decode linear: "gemv", "linear" (F.linear on the BF16
    weight) or "w8a16" (the INT8-weight GEMM). fmt is the stored weight's format: "bf16", "int8" or "int4"."""
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
    if fmt not in ("bf16", "int8", "int4"):
        raise ValueError(f"weight format must be bf16, int8 or int4, got {fmt!r}")
    if mode == "cublas":
        return "linear"
    if fmt == "bf16":
        return "gemv" if B <= BF16_GEMV_MAX_BATCH or (B <= GEMV_MAX_BATCH and K < 8192) else "linear"
    if B <= GEMV_MAX_BATCH:
        return "gemv"
    if fmt == "int8":
        if K >= 8192 and B <= 24 and has_bf16:
            return "linear"
        if N < W8A16_MIN_ROWS and K < 8192 and B <= GEMV_MAX_BATCH_NARROW:
            return "gemv"
        if has_bf16 and B > (W8A16_MAX_BATCH // 2 if N >= HEAD_ROWS else W8A16_MAX_BATCH):
            return "linear"
        return "w8a16"
    # INT4: the GEMV (16-row chunks, a quarter of the BF16 bytes) while it beats F.linear on the kept copy
    if not has_bf16:
        return "gemv"
    if K >= 8192:
        return "linear"
    return "gemv" if B <= (48 if N >= HEAD_ROWS else 24 if N >= W8A16_MIN_ROWS else GEMV_MAX_BATCH_NARROW) else "linear"


class DecodeLinears:
    """The decode linears of one model, keyed like the reference's `lin` dict (("qkv", i), ("w13", i), ("head", 0),
    ...; w1|w3 stacked as one [2 I, K] matrix under a "w13" key).

    weights: {key: BF16 [N, K]} on the GPU. w4_pre: {key: (packed uint8 [N, K/2], scales fp32 [N, K/group])
    (the reference's format), optionally + inv_s [K]} or {key: (qweight int32 [N, K/8], scales fp16, qzeros int32)
    (GPTQ-style), optionally + inv_s}. w4_clip: INT4 scales by the clip search of quantize_int4 (runtime.py:186).
    drop_bf16 frees the BF16 copies the quantized weights no longer need
    (runtime.py:200-215); it requires mode "int8" as in the reference (runtime.py:33-34)."""

    def __init__(self, weights, gemv="int8", w4_group=GROUP, w4_keep_int8=(), w4_pre=None, drop_bf16=False,
                 w4_clip=False):
        if gemv not in MODES:
            raise ValueError(f"gemv must be one of {MODES}, got {gemv!r}")
        if drop_bf16 and gemv != "int8":
            raise ValueError("drop_bf16 needs INT8 decode weights (the W8A16 GEMM replaces the BF16 copies)")
        self.mode, self.drop_bf16 = gemv, drop_bf16
        self.K = ext()
        self.epilogue_fusion = os.environ.get("LFM2_EPI", "1") != "0"  # runtime.py:35; 0 = separate ops
        # the batch-1 GEMVs that normalize their input row themselves (gemv_rmsnorm); 0 = add_rmsnorm_q, then the GEMV
        self.norm_fusion = os.environ.get("LFM2_NORM_GEMV", "1") != "0"
        self.last_path = None
        self.lin, self.lin_scale, self.lin_zeros, self.lin_inv_s, self.lin_bf16, self.w8 = {}, {}, {}, {}, {}, {}
        w4_pre = w4_pre or {}
        keep = set(w4_keep_int8)
        for key, w in weights.items():
            if w.dtype != torch.bfloat16 or w.dim() != 2 or not w.is_cuda:
                raise ValueError(f"weight {key}: BF16 [N, K] on the GPU")
            if gemv in ("cublas", "bf16"):
                self.lin[key] = w.contiguous()
                continue
            self.lin_bf16[key] = w
            if gemv == "int8" or key[0] in keep:  # runtime.py:178-179
                self.lin[key], self.lin_scale[key] = quantize_int8(w)
            elif key in w4_pre:  # runtime.py:180-181, with the AWQ inv_s of :183-184 carried along
                self._set_w4_pre(key, w, w4_pre[key])
            else:
                self.lin[key], self.lin_scale[key] = quantize_int4(w, w4_group, w4_clip)
            if self.lin[key].dtype == torch.int8:
                self.w8[key] = Int8Linear(q=self.lin[key], scale=self.lin_scale[key], a8=False)
        if drop_bf16:
            self.lin_bf16 = {}

    def _set_w4_pre(self, key, w, pre):
        pre = tuple(pre)
        fmt_gptq = pre[0].dtype == torch.int32
        n = 3 if fmt_gptq else 2
        if len(pre) not in (n, n + 1):
            raise ValueError(f"w4_pre[{key}]: (packed, scales[, inv_s]) or (qweight, scales, qzeros[, inv_s])")
        N, K = w.shape
        if tuple(pre[0].shape) != ((N, K // 8) if fmt_gptq else (N, K // 2)):
            raise ValueError(f"w4_pre[{key}]: packed weight shape {tuple(pre[0].shape)} does not match [{N}, {K}]")
        self.lin[key], self.lin_scale[key] = pre[0], pre[1]
        if fmt_gptq:
            self.lin_zeros[key] = pre[2]
        if len(pre) == n + 1:
            inv_s = pre[n]
            if inv_s.numel() != K:
                raise ValueError(f"w4_pre[{key}]: inv_s must have K = {K} elements")
            self.lin_inv_s[key] = inv_s.reshape(K)

    # ---- dispatch -----------------------------------------------------------------------------------------------
    def fmt(self, key):
        dt = self.lin[key].dtype
        return "bf16" if dt == torch.bfloat16 else "int8" if dt == torch.int8 else "int4"

    def shape(self, key):
        """(N, K) of the weight behind key."""
        w = self.lin[key]
        return w.shape[0], w.shape[1] * {torch.bfloat16: 1, torch.int8: 1, torch.uint8: 2, torch.int32: 8}[w.dtype]

    def path(self, B, key):
        N, K = self.shape(key)
        return linear_path(self.mode, self.fmt(key), B, N, K, key in self.lin_bf16)

    def _bf16_weight(self, key):
        w = self.lin[key]
        return w if w.dtype == torch.bfloat16 else self.lin_bf16[key]

    def _gemv(self, x, key, y, epi):
        """The GEMV for key into y, epilogue epi (0 none, 1 SwiGLU over w1|w3, 2 residual add into y)."""
        w, fmt = self.lin[key], self.fmt(key)
        if fmt == "int4":
            inv_s = self.lin_inv_s.get(key)
            if inv_s is not None:  # AWQ: the weight columns were scaled by s, so x is scaled by 1/s
                x = x * inv_s.to(x.dtype)
            if w.dtype == torch.int32:
                self.K.gemv_w4z(w, self.lin_scale[key], self.lin_zeros[key], x, y, epi=epi)
            else:
                self.K.gemv_w4(w, self.lin_scale[key], x, y, epi=epi)
        elif epi == 1:
            self.K.gemv_epi(0, w, self.lin_scale.get(key), x, y)
        elif epi == 2:
            self.K.gemv_residual(w, self.lin_scale.get(key), x, y)
        else:
            self.K.gemv(w, self.lin_scale.get(key), x, y)

    # ---- the reference's _linear and its fused call sites -------------------------------------------------------
    def linear(self, x, key, bias=None):
        """y [B, N] = x [B, K] @ W^T (+ bias), through the path linear_path picks (runtime.py:223-244)."""
        B = x.shape[0]
        p = self.last_path = self.path(B, key)
        if p == "linear":
            return F.linear(x, self._bf16_weight(key), bias)
        if p == "w8a16":
            y = self.w8[key](x)
            return y if bias is None else y + bias
        y = torch.empty(B, self.lin[key].shape[0], device=x.device, dtype=x.dtype)
        self._gemv(x.contiguous(), key, y, 0)
        return y if bias is None else y + bias

    def swiglu(self, x, key, out=None):
        """act [B, I] = bf16(silu(g) * u) with [g | u] = x @ W13^T: the GEMV's fused epilogue on the GEMV path,
        else the linear followed by silu_mul (runtime.py:277-282)."""
        B = x.shape[0]
        N = self.lin[key].shape[0]
        act = out if out is not None else torch.empty(B, N // 2, device=x.device, dtype=x.dtype)
        if self.epilogue_fusion and self.path(B, key) == "gemv":
            self.last_path = "gemv"
            self._gemv(x.contiguous(), key, act, 1)
        else:
            g = self.linear(x, key)
            self.K.silu_mul(g, act)
        return act

    def norm_fusable(self, B, key):
        """Whether the linear for key at batch B runs as one GEMV that also computes its input's RMSNorm
        (gemv_rmsnorm): batch 1 on the GEMV path, INT8 or BF16 weights, K a supported chunk multiple."""
        if not (self.norm_fusion and B == 1 and self.path(B, key) == "gemv"):
            return False
        fmt = self.fmt(key)
        K = self.shape(key)[1]
        if fmt == "int8":
            return K in (1024, 2048, 4096, 8192)
        return fmt == "bf16" and K in (512, 1024, 2048, 4096)

    def linear_normed(self, h, key, norm_w, eps, swiglu=False, out=None):
        """linear(rms_norm(h) * norm_w, key), or swiglu(...) of it, as one GEMV (norm_fusable(1, key) must hold):
        bit-identical to add_rmsnorm_q's x followed by the GEMV."""
        w = self.lin[key]
        N = w.shape[0] // 2 if swiglu else w.shape[0]
        y = out if out is not None else torch.empty(1, N, device=h.device, dtype=h.dtype)
        self.last_path = "gemv"
        self.K.gemv_rmsnorm(w, self.lin_scale.get(key), h.contiguous(), norm_w, eps, y, 1 if swiglu else 0)
        return y

    def residual(self, x, key, h):
        """h [B, N] = bf16(h + bf16(x @ W^T)) in place: the GEMV's fused residual epilogue on the GEMV path, else the
        linear and a BF16 add (the rounding of the residual add in the reference's add_rmsnorm)."""
        B = x.shape[0]
        if self.epilogue_fusion and self.path(B, key) == "gemv":
            self.last_path = "gemv"
            self._gemv(x.contiguous(), key, h, 2)
        else:
            h.add_(self.linear(x, key))
        return h
