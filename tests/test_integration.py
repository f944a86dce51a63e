"""The binding INTEGRATION.md prescribes for the reference stack: its code block is executed as printed (with _ROOT
pointed at this checkout), loading this package as `lfm2q_ops` next to -- not in place of -- an `lfm2opt` package;
the ops and the decode dispatch are then driven through that name (on the GPU in the marked test)."""

import re
import sys

import pytest

from conftest import PKG, ROOT


def binding_block():
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    block = next(b for b in blocks if "spec_from_file_location" in b)
    return re.sub(r'^_ROOT = ".*"$', f'_ROOT = "{PKG / "lfm2opt"}"', block, count=1, flags=re.M)


@pytest.fixture(scope="module")
def ns():
    for name in [m for m in sys.modules if m == "lfm2q_ops" or m.startswith("lfm2q_ops.")]:
        del sys.modules[name]
    env = {}
    exec(compile(binding_block(), "INTEGRATION.md", "exec"), env)
    return env


def test_binding_loads_under_its_own_name(ns):
    import lfm2opt.kernels

    mod = sys.modules["lfm2q_ops"]
    assert ns["lfm2q_ops"] is mod
    assert mod.kernels is not lfm2opt.kernels  # a separate package instance; the reference's name is untouched
    assert ns["mm_ext"] is mod.kernels.ext and ns["int8_ext"] is mod.kernels.int8_ext
    E, E8 = ns["mm_ext"](), ns["int8_ext"]()
    for op in ("gemv", "gemv_w4", "gemv_w4z", "gemv_epi", "gemv_residual", "silu_mul", "set_pdl", "set_gemv_impl"):
        assert callable(getattr(E, op)), op
    for op in ("gemm_i8", "gemm_i8_q", "gemm_w8", "gemm_i8_i32", "quant_rows", "add_rmsnorm_q", "add_layernorm_q",
               "silu_mul_q"):
        assert callable(getattr(E8, op)), op


def test_decode_dispatch_through_binding(ns):
    from lfm2q_ops.decode import DecodeLinears, linear_path  # noqa: F401  (importable by the bound name)
    from lfm2q_ops.int8 import Int8Linear, act_group  # noqa: F401

    assert linear_path("int8", "int8", 1, 16384, 2048, True) == "gemv"
    assert linear_path("int8", "int8", 64, 65536, 2048, True) == "w8a16"


def test_runtime_through_binding(ns):
    """The decode runtime of the integration section resolves under the bound name, its imports included."""
    from lfm2q_ops.runtime import StaticDecoder, decode_weight_modules, load_decode_weights  # noqa: F401

    assert StaticDecoder.generate.__qualname__ == "StaticDecoder.generate"


@pytest.mark.gpu
def test_binding_runs_decode_linears(ns, cuda):
    """DecodeLinears built through the bound name quantizes and runs the SwiGLU and residual GEMVs at batch 1, the
    same bits as the ops called through this package's own name."""
    import torch
    from lfm2q_ops.decode import DecodeLinears

    from lfm2opt.kernels import ext

    g = torch.Generator(device="cuda").manual_seed(11)
    w13 = (torch.randn(2 * 512, 1024, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(1024, 512, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    dl = DecodeLinears({("w13", 0): w13, ("w2", 0): w2}, gemv="int8")
    x = torch.randn(1, 1024, device="cuda", generator=g).to(torch.bfloat16)
    h = torch.randn(1, 1024, device="cuda", generator=g).to(torch.bfloat16)
    act = dl.swiglu(x, ("w13", 0))
    h1 = dl.residual(act, ("w2", 0), h.clone())
    E = ext()
    act_ref = torch.empty(1, 512, device="cuda", dtype=torch.bfloat16)
    E.gemv_epi(0, dl.lin[("w13", 0)], dl.lin_scale[("w13", 0)], x, act_ref)
    h_ref = h.clone()
    E.gemv_residual(dl.lin[("w2", 0)], dl.lin_scale[("w2", 0)], act_ref, h_ref)
    assert torch.equal(act, act_ref) and torch.equal(h1, h_ref)
