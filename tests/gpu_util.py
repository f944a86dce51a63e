"""Helpers shared by the GPU tests: numpy <-> torch device tensors and the error metrics of the parity bar."""

import numpy as np
import torch


def dev_bf16(a, device="cuda"):
    """numpy uint16 bf16 bits -> torch bf16 tensor on the device."""
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def dev(a, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host_bits(t):
    """torch bf16 tensor -> numpy uint16 bits."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_to_f64(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def ulp_dist(a, b):
    ia = np.asarray(a, np.uint16).astype(np.int64)
    ib = np.asarray(b, np.uint16).astype(np.int64)
    ia = np.where(ia >= 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib >= 0x8000, 0x8000 - ib, ib)
    return np.abs(ia - ib)


def rel_err(out_bits, ref_bits):
    """(max |out - ref| / max |ref|, mean |out - ref|, max bf16 ulps) -- the bf16 parity bar's three numbers."""
    o, r = bf16_to_f64(out_bits), bf16_to_f64(ref_bits)
    d = np.abs(o - r)
    return float(d.max() / max(np.abs(r).max(), 1e-30)), float(d.mean()), int(ulp_dist(out_bits, ref_bits).max())


def assert_close_bf16(out_bits, ref_bits, tol=1e-2, what=""):
    """max |err| / max |ref| <= tol (the stated bf16 tolerance); the mean abs error is reported."""
    mx, mean, ul = rel_err(out_bits, ref_bits)
    print(f"{what}: max rel err {mx:.3e}, mean abs err {mean:.3e}, max {ul} bf16 ulp")
    assert mx <= tol, f"{what}: max rel err {mx:.3e} > {tol}"
