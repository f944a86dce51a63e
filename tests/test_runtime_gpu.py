"""The decode runtime (lfm2opt.runtime.StaticDecoder) on MI355X: a six-layer LFM2 model (four short-conv, two
attention layers; random weights, transformers' Lfm2ForCausalLM) decoded with every linear on the library's kernels,
the step captured as a HIP graph.

Parity bar: the logits at every position of a 21-token sequence (fed one token per step) within max |err| / max
|ref| <= 4e-2 of transformers' fp32 forward on the CPU over the same sequence, run on the weights the GPU paths read
(the dequantized INT8 / INT4 weights where a GEMV or W8A16 ran, the BF16 ones where F.linear or the BF16 GEMV ran)
and on the GPU model's BF16 embeddings and norms. The bar covers the bf16 rounding of the activations between the
ops: the same step with bf16 activations and fp32-exact linears on the CPU lands 1.4 % from that forward. Graph
replays and eager steps give bit-identical logits, and graph and eager generate() the same tokens."""

import copy

import pytest
import torch

from lfm2_tiny import reference_logits, step_logits, tiny_lfm2

pytestmark = pytest.mark.gpu

TOL = 4e-2


@pytest.fixture(scope="module")
def nets(cuda):
    net = tiny_lfm2(seed=21)
    return net, copy.deepcopy(net).to(cuda, torch.bfloat16)


def path_weight(lin, key, B):
    """The fp32 weight (CPU) that the call for key at batch B multiplies."""
    from lfm2opt.quant import dequantize_int4

    p = lin.path(B, key)
    w = lin.lin[key]
    if p == "linear" or lin.fmt(key) == "bf16":
        return lin._bf16_weight(key).float().cpu()
    if lin.fmt(key) == "int8":
        return (w.float() * lin.lin_scale[key].float()[:, None]).cpu()
    return dequantize_int4(w, lin.lin_scale[key]).float().cpu()


def oracle(gpu_net, dec, B):
    """fp32 CPU copy of the GPU model whose decode linears hold the weights the GPU paths read at batch B; the head
    gets its own copy (the token embedding it is tied to keeps the BF16 table the step reads)."""
    from lfm2opt.runtime import decode_weight_modules

    ref = copy.deepcopy(gpu_net).to("cpu", torch.float32)
    mods = dict(ref.named_modules())
    for key, names in decode_weight_modules(ref).items():
        W = path_weight(dec.lin, key, B)
        r0 = 0
        for n in names:
            m = mods[n]
            rows = m.weight.shape[0]
            m.weight = torch.nn.Parameter(W[r0:r0 + rows].clone(), requires_grad=False)
            r0 += rows
        assert r0 == W.shape[0]
    return ref


def rel_err(a, b):
    return float((a - b).abs().max() / b.abs().max())


@pytest.mark.parametrize("mode,B,paths", [("int8", 2, {"gemv"}), ("int4", 2, {"gemv"}), ("bf16", 2, {"gemv"}),
                                          ("cublas", 2, {"linear"}), ("int8", 40, {"w8a16"}),
                                          ("int4", 20, {"linear"})])
def test_decode_step_against_transformers(nets, mode, B, paths):
    from lfm2opt.runtime import StaticDecoder

    _, gnet = nets
    dec = StaticDecoder(gnet, bucket=32, keep_logits=True, gemv=mode)
    taken = {dec.lin.path(B, key) for key in dec.lin.lin}
    assert taken == paths
    ids = torch.randint(0, gnet.config.vocab_size, (B, 21), generator=torch.Generator().manual_seed(B))
    print(f"runtime {mode} B={B}", flush=True)
    got = step_logits(dec, ids, graph=True)
    eager = step_logits(dec, ids, graph=False)
    assert torch.equal(got, eager), "graph replays differ from eager steps"
    want = reference_logits(oracle(gnet, dec, B), ids)
    err = rel_err(got, want)
    print(f"runtime {mode} B={B}: max |err| / max |ref| = {err:.2e}")
    assert err <= TOL


def test_generate_graph_equals_eager(nets):
    from lfm2opt.runtime import StaticDecoder

    _, gnet = nets
    dec = StaticDecoder(gnet, bucket=32, gemv="int8")
    ids = torch.randint(3, gnet.config.vocab_size, (3, 7), generator=torch.Generator().manual_seed(2))
    a = dec.generate(ids, 12)
    b = dec.generate(ids, 12, graph=False)
    assert a.shape == (3, 19) and torch.equal(a, b)
    assert torch.equal(dec.generate(ids, 12), a)  # a second request on the same captured graph


def test_drop_bf16_frees_the_module_weights(cuda):
    """drop_bf16: the HF linears' own weights are freed, the tied head's table stays (the step's embedding), and
    decoding runs on the INT8 weights alone (W8A16 above the GEMV's batches)."""
    from lfm2opt.runtime import StaticDecoder

    gnet = copy.deepcopy(tiny_lfm2(seed=23)).to(cuda, torch.bfloat16)
    dec = StaticDecoder(gnet, bucket=32, keep_logits=True, gemv="int8", drop_bf16=True)
    assert gnet.model.layers[0].feed_forward.w1.weight.numel() == 0 and gnet.model.embed_tokens.weight.numel() > 0
    assert not dec.lin.lin_bf16
    ids = torch.randint(0, gnet.config.vocab_size, (40, 9), generator=torch.Generator().manual_seed(5))
    assert {dec.lin.path(40, key) for key in dec.lin.lin} == {"w8a16"}
    got = step_logits(dec, ids, graph=True)
    ref_net = tiny_lfm2(seed=23)  # the same weights again (deterministic init), to hold the dequantized linears
    ref_net = copy.deepcopy(ref_net).to(torch.bfloat16).to(torch.float32)
    mods = dict(ref_net.named_modules())
    from lfm2opt.runtime import decode_weight_modules

    for key, names in decode_weight_modules(ref_net).items():
        W = path_weight(dec.lin, key, 40)
        r0 = 0
        for n in names:
            rows = mods[n].weight.shape[0]
            mods[n].weight = torch.nn.Parameter(W[r0:r0 + rows].clone(), requires_grad=False)
            r0 += rows
    assert rel_err(got, reference_logits(ref_net, ids)) <= TOL
