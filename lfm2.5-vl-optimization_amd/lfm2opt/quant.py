"""Weight formats of the decode GEMVs and the W8A8 GEMM, computed with torch on the weight's own device (load-time
work, not on the hot path).

* INT8: one fp32 scale per output row, W ~= q * s[n], q in [-127, 127] (src/lfm2opt/quant.py:13-18).
* INT4, symmetric: one fp32 scale per group of `group` inputs, q in [-8, 7] stored as q + 8, two per byte with
  element 2j in the low nibble (src/lfm2opt/quant.py:21-47, gptq.py:164-169). Read as little-endian int32 words the
  same bytes are [N, K/8] with nibble i of word w holding k = 8 w + i.
* INT4, GPTQ-style asymmetric: q in [0, 15] packed 8 per int32 along K ([N, K/8], nibble i of word w = k 8w + i),
  fp16 scales [N, K/group], 4-bit zero points packed 8 per int32 ([N, ceil(G/8)], nibble j of word w = group
  8w + j); W ~= s (q - z). The symmetric format is the case z = 8.
"""

import torch

GROUP = 128


@torch.no_grad()
def quantize_int8(w: torch.Tensor):
    """(q int8 [N, K], scale fp32 [N]); scale = max(|w_n|) / 127 floored at 1e-12, q = round(w / scale)."""
    wf = w.float()
    scale = (wf.abs().amax(1) / 127).clamp_min(1e-12)
    q = torch.round(wf / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return q.contiguous(), scale.contiguous()


CLIP_FRACTIONS = torch.linspace(0.70, 1.00, 16)  # clip search: candidate scales absmax * a / 7
CLIP_ROWS = 1024  # clip search: weight rows per pass (16 candidates x rows x K fp32 values live at once)


def _clip_scales(wg: torch.Tensor, amax: torch.Tensor):
    """Per group, the candidate scale amax * a / 7 (a in CLIP_FRACTIONS) whose round-to-nearest INT4 reconstruction
    has the smallest squared error; the first such candidate on ties. wg [n, G, group], amax [n, G]."""
    out = torch.empty_like(amax)
    cand = CLIP_FRACTIONS.to(wg.device)[:, None, None]
    for r0 in range(0, wg.shape[0], CLIP_ROWS):
        w = wg[r0:r0 + CLIP_ROWS]
        s = amax[None, r0:r0 + CLIP_ROWS] * cand / 7                          # [16, n, G]
        rec = torch.round(w[None] / s[..., None]).clamp(-8, 7) * s[..., None]  # [16, n, G, group]
        err = (rec - w[None]).pow(2).sum(-1)                                  # [16, n, G]
        best = err.argmin(0, keepdim=True)                                     # first minimum
        out[r0:r0 + CLIP_ROWS] = s.gather(0, best)[0]
    return out


@torch.no_grad()
def quantize_int4(w: torch.Tensor, group: int = GROUP, clip_search: bool = False):
    """Symmetric round-to-nearest INT4: (packed uint8 [N, K/2], scale fp32 [N, K/group]); scale = amax / 7, or with
    clip_search the scale amax * a / 7, a in 0.70 .. 1.00 (16 steps), with the smallest squared reconstruction error
    of its group (reference: src/lfm2opt/quant.py:21-39)."""
    N, K = w.shape
    assert K % group == 0
    wg = w.float().view(N, K // group, group)
    amax = wg.abs().amax(-1).clamp_min(1e-12)
    scale = _clip_scales(wg, amax) if clip_search else amax / 7
    q = torch.round(wg / scale[..., None]).clamp(-8, 7).to(torch.int16).view(N, K) + 8
    return ((q[:, 0::2] | (q[:, 1::2] << 4)).to(torch.uint8).contiguous(), scale.contiguous())


@torch.no_grad()
def dequantize_int4(packed: torch.Tensor, scale: torch.Tensor):
    """fp32 [N, K] from the symmetric format: (nibble - 8) * scale[n, k // group]."""
    p = packed.to(torch.int16)
    q = torch.stack([(p & 0xF) - 8, (p >> 4) - 8], dim=-1).view(packed.shape[0], -1).float()
    group = q.shape[1] // scale.shape[1]
    return (q.view(q.shape[0], -1, group) * scale[..., None]).view(q.shape[0], -1)


def pack_int4(Wq, scales):
    """Dequantized symmetric INT4 weights + their scales -> (packed uint8 [N, K/2], scales) (gptq.py:164-169)."""
    N, K = Wq.shape
    group = K // scales.shape[1]
    q = torch.round(Wq.view(N, K // group, group) / scales[..., None]).clamp(-8, 7).to(torch.int16).view(N, K) + 8
    return (q[:, 0::2] | (q[:, 1::2] << 4)).to(torch.uint8).contiguous(), scales.contiguous()


def _pack_nibbles(v: torch.Tensor):
    """int [R, C] with values 0..15, C padded up to a multiple of 8 -> int32 [R, ceil(C/8)], nibble i of word w =
    element 8 w + i."""
    R, C = v.shape
    Cp = (C + 7) // 8 * 8
    if Cp != C:
        v = torch.nn.functional.pad(v, (0, Cp - C))
    v = v.to(torch.int64).view(R, Cp // 8, 8)
    shifts = torch.arange(0, 32, 4, device=v.device, dtype=torch.int64)
    words = (v << shifts).sum(-1)
    return torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32).contiguous()


def _unpack_nibbles(words: torch.Tensor, C: int):
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(0, 32, 4, device=w.device, dtype=torch.int64)
    return ((w[..., None] >> shifts) & 15).view(words.shape[0], -1)[:, :C]


@torch.no_grad()
def pack_int4_zp(q: torch.Tensor, z: torch.Tensor):
    """q int [N, K] in [0, 15], z int [N, G] in [0, 15] -> (qweight int32 [N, K/8], qzeros int32 [N, ceil(G/8)])."""
    return _pack_nibbles(q), _pack_nibbles(z)


@torch.no_grad()
def quantize_int4_zp(w: torch.Tensor, group: int = GROUP):
    """Asymmetric min/max INT4 (GPTQ storage, no act-order): (qweight int32 [N, K/8], scales fp16 [N, K/group],
    qzeros int32 [N, ceil(G/8)]) with s = (max - min) / 15, z = round(-min / s), q = clamp(round(w / s) + z)."""
    N, K = w.shape
    assert K % group == 0 and K % 8 == 0
    wg = w.float().view(N, K // group, group)
    lo, hi = wg.amin(-1).clamp_max(0), wg.amax(-1).clamp_min(0)
    s = ((hi - lo) / 15).clamp_min(1e-8).to(torch.float16)
    sf = s.float()
    z = torch.round(-lo / sf).clamp(0, 15)
    q = (torch.round(wg / sf[..., None]) + z[..., None]).clamp(0, 15).view(N, K)
    qw, qz = pack_int4_zp(q.to(torch.int32), z.to(torch.int32))
    return qw, s.contiguous(), qz


@torch.no_grad()
def dequantize_int4_zp(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor):
    """fp32 [N, K] = s[n, g] (q - z[n, g]) from the GPTQ-style format."""
    N = qweight.shape[0]
    K = qweight.shape[1] * 8
    G = scales.shape[1]
    group = K // G
    q = _unpack_nibbles(qweight, K).float()
    z = _unpack_nibbles(qzeros, G).float()
    return ((q.view(N, G, group) - z[..., None]) * scales.float()[..., None]).view(N, K)
