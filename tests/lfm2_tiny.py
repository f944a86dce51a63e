"""Small LFM2 language models (transformers' Lfm2ForCausalLM, random weights) for the decode runtime's tests, and an
F.linear stand-in for DecodeLinears."""

import torch
import torch.nn.functional as F


def tiny_lfm2(seed=0, layer_types=("conv", "conv", "full_attention", "conv", "full_attention", "conv"),
              hidden=256, heads=4, kv_heads=2, ffn=768, vocab=1024, conv_bias=False):
    """An fp32 Lfm2ForCausalLM on the CPU: linears N(0, 0.02) as transformers initializes them, and -- unlike
    transformers' init, which sets them to 1 / leaves the conv as is -- every RMSNorm weight 1 + N(0, 0.1) and the conv
    taps N(0, 0.3), so that a dropped or misplaced weight changes the result. ffn is the config's intermediate size
    (auto-adjusted to 2/3, rounded up to 256, as the LFM2 configs ask)."""
    from transformers import Lfm2Config, Lfm2ForCausalLM

    cfg = Lfm2Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=ffn, num_hidden_layers=len(layer_types),
                     num_attention_heads=heads, num_key_value_heads=kv_heads, layer_types=list(layer_types),
                     max_position_embeddings=512, norm_eps=1e-5, conv_bias=conv_bias, tie_word_embeddings=True)
    torch.manual_seed(seed)
    net = Lfm2ForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in net.named_parameters():
            if name.endswith("norm.weight") or name.endswith("layernorm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            elif name.endswith("conv.conv.weight"):
                p.copy_(0.3 * torch.randn(p.shape, generator=g))
            elif name.endswith(".bias"):
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
    return net


class TorchLinears:
    """DecodeLinears' interface on F.linear over {key: weight} (any device and dtype): the SwiGLU as
    silu(g) * u in the weights' dtype, the residual as h += x W^T."""

    def __init__(self, weights):
        self.w = weights
        self.last_path = "linear"

    def linear(self, x, key, bias=None):
        return F.linear(x, self.w[key], bias)

    def swiglu(self, x, key, out=None):
        g = F.linear(x, self.w[key])
        i = g.shape[-1] // 2
        return F.silu(g[:, :i]) * g[:, i:]

    def residual(self, x, key, h):
        return h.add_(F.linear(x, self.w[key]))


def reference_logits(net, ids):
    """transformers' own forward over the whole sequence: logits [B, T, V] in fp32 (the model's eager path on the
    CPU; no cache, causal mask)."""
    with torch.no_grad():
        return net(input_ids=ids, use_cache=False).logits.float()


def step_logits(dec, ids, graph=False):
    """The runtime's logits at every position of ids [B, T]: the prompt fed one token per decode step (teacher
    forcing), each step's logits read from the state's logits buffer. [B, T, V] fp32 on the CPU."""
    B, T = ids.shape
    st = dec.state(B, T + 1, 1, graph)
    out = []
    dev_ids = ids.to(dec.device)
    for t in range(T):
        st.tok.copy_(dev_ids[:, t])
        st.row.zero_()
        st.graph.replay() if graph else dec._step(st)
        out.append(st.logits.cpu().clone())
    return torch.stack(out, dim=1)
