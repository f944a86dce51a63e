"""The decode runtime (lfm2opt.runtime) on the CPU: its step math against transformers' own LFM2 forward, its weight
keys against the reference's, and the on-disk decode-weight format.

The step is checked with an F.linear stand-in for DecodeLinears (the library's kernels need a GPU), in fp32, feeding
a token sequence one position per step: the logits at every position must equal transformers' Lfm2ForCausalLM
forward over the whole sequence (its causal attention, RMSNorms, rotary embedding and short conv) to fp32 rounding.
This pins the restated non-matmul ops -- a rotary embedding at the wrong position, a cache slot written or masked
wrongly, a conv state shifted the wrong way, a norm weight dropped -- at every layer type and position."""

import pytest
import torch

from lfm2_tiny import TorchLinears, reference_logits, step_logits, tiny_lfm2

from lfm2opt.runtime import (StaticDecoder, decode_weight_modules, decode_weights, load_decode_weights,
                             save_decode_weights)


def rel_err(a, b):
    return float((a - b).abs().max() / b.abs().max())


@pytest.mark.parametrize("conv_bias", [False, True])
def test_step_matches_transformers_forward(conv_bias):
    net = tiny_lfm2(seed=3, conv_bias=conv_bias)
    dec = StaticDecoder(net, bucket=16, keep_logits=True, linears=TorchLinears(decode_weights(net)))
    ids = torch.randint(0, net.config.vocab_size, (2, 21), generator=torch.Generator().manual_seed(4))
    got, want = step_logits(dec, ids), reference_logits(net, ids)
    assert rel_err(got, want) < 1e-5


def test_step_catches_a_planted_mistake():
    """The comparison above fails when the restated math is wrong: the rotary embedding taken at position 0 for
    every step (a cache-position bug) moves the logits far beyond the bar."""
    net = tiny_lfm2(seed=5)
    dec = StaticDecoder(net, bucket=16, keep_logits=True, linears=TorchLinears(decode_weights(net)))
    ids = torch.randint(0, net.config.vocab_size, (1, 9), generator=torch.Generator().manual_seed(6))
    want = reference_logits(net, ids)
    dec.inv_freq = dec.inv_freq * 0  # every position rotated as position 0
    assert rel_err(step_logits(dec, ids), want) > 1e-2


def test_generate_is_greedy_decoding_of_the_forward():
    """generate(): the prompt through the step, then greedy tokens; each new token is the argmax of transformers'
    forward over everything before it (EOS masked, as the fixed-length default asks)."""
    net = tiny_lfm2(seed=7)
    dec = StaticDecoder(net, bucket=16, linears=TorchLinears(decode_weights(net)))
    ids = torch.randint(3, net.config.vocab_size, (2, 6), generator=torch.Generator().manual_seed(8))
    out = dec.generate(ids, 5, graph=False)
    assert out.shape == (2, 11) and torch.equal(out[:, :6], ids)
    for t in range(6, 11):
        logits = reference_logits(net, out[:, :t])[:, -1]
        logits[:, dec.eos] = float("-inf")
        assert torch.equal(out[:, t], logits.argmax(-1))


def test_generate_requests():
    net = tiny_lfm2(seed=9, layer_types=("conv", "full_attention"))
    dec = StaticDecoder(net, bucket=8, linears=TorchLinears(decode_weights(net)))
    ids = torch.randint(3, net.config.vocab_size, (1, 4), generator=torch.Generator().manual_seed(1))
    assert dec.generate(ids, 1, graph=False).shape == (1, 5)
    assert torch.equal(dec.generate(ids, 0, graph=False), dec.generate(ids, 1, graph=False))  # at least one token
    a = dec.generate(ids, 6, graph=False)
    assert torch.equal(dec.generate(ids, 6, graph=False), a)  # state reset between requests
    with pytest.raises(ValueError, match="padded batch takes input_ids"):
        dec.prefill(ids, 2, attention_mask=torch.tensor([[0, 1, 1, 1]]), graph=False,
                    inputs_embeds=net.model.embed_tokens(ids).detach())
    with pytest.raises(ValueError, match="at least one"):
        dec.prefill(ids[:, :0], 2, graph=False)


def test_batched_prefill_leaves_the_state_of_the_step():
    """fused_prefill on the CPU model: the last position's logits equal transformers' forward, and the key / value
    caches and conv rings it leaves equal those of the prompt run through the step one position per step, at prompt
    lengths covering every ring offset (T mod L) and a prompt shorter than L; generation then continues the same.
    The prompt attention is taken in one block and (blocks_from = 4) in four blocks of uneven sizes."""
    net = tiny_lfm2(seed=4, conv_bias=True)
    lin = TorchLinears(decode_weights(net))
    assert net.config.conv_L_cache == 3
    for T, blocks_from in ((1, 1024), (2, 1024), (5, 1024), (7, 1024), (5, 4), (7, 4), (11, 4)):
        ids = torch.randint(3, net.config.vocab_size, (2, T), generator=torch.Generator().manual_seed(T))
        fused = StaticDecoder(net, bucket=16, keep_logits=True, fused_prefill=True, linears=lin)
        fused.prompt_blocks_from = blocks_from
        first, s = fused.prefill(ids, 4, graph=False)
        assert rel_err(fused.last_prefill_logits, reference_logits(net, ids)[:, -1]) < 1e-5
        step = StaticDecoder(net, bucket=16, linears=lin)
        first2, s2 = step.prefill(ids, 4, graph=False)
        assert torch.equal(first, first2) and s.ctr.tolist() == s2.ctr.tolist() == [T, 1]
        for name in ("k", "v", "conv"):
            for i, buf in getattr(s, name).items():
                assert rel_err(buf, getattr(s2, name)[i]) < 1e-5, (T, name, i)
        assert torch.equal(fused.generate(ids, 4, graph=False), step.generate(ids, 4, graph=False))


@pytest.mark.parametrize("T,pad", [(2, 1), (5, 2), (6, 3), (8, 4)])
def test_padded_batch_prefill(T, pad):
    """A left-padded batch (runtime.py:440-460): the prompt runs through transformers' forward with the mask and its
    cache is copied into the static buffers. Row 0 (no padding) must leave exactly the caches and conv ring of the
    same prompt prefilled alone through the step -- keys transposed, conv state rows at their ring positions, for
    prompts shorter than the conv length and at every ring offset -- and generate the same tokens; both rows' first
    tokens are the argmax of the masked forward (EOS blocked). A mask of all ones takes the ordinary path."""
    net = tiny_lfm2(seed=21, conv_bias=True)
    lin = TorchLinears(decode_weights(net))
    assert net.config.conv_L_cache == 3
    g = torch.Generator().manual_seed(T * 10 + pad)
    ids = torch.randint(3, net.config.vocab_size, (2, T), generator=g)
    mask = torch.ones(2, T, dtype=torch.long)
    mask[1, :pad] = 0
    dec = StaticDecoder(net, bucket=16, keep_logits=True, linears=lin)
    first, st = dec.prefill(ids, 4, attention_mask=mask, graph=False)
    with torch.no_grad():
        want = net(input_ids=ids, attention_mask=mask, use_cache=False).logits.float()[:, -1]
    assert rel_err(dec.last_prefill_logits, want) < 1e-5
    want[:, dec.eos] = float("-inf")
    assert torch.equal(first, want.argmax(-1)) and st.ctr.tolist() == [T, 1]
    alone = StaticDecoder(net, bucket=16, linears=lin)
    first0, s0 = alone.prefill(ids[:1], 4, graph=False)
    assert torch.equal(first[:1], first0)
    for name in ("k", "v", "conv"):
        for i, buf in getattr(st, name).items():
            row0 = buf[:, :1] if name == "conv" else buf[:1]
            assert rel_err(row0, getattr(s0, name)[i]) < 1e-5, (name, i)
    out = dec.generate(ids, 4, attention_mask=mask, graph=False)
    assert torch.equal(out[:1], alone.generate(ids[:1], 4, graph=False))
    full = torch.ones(2, T, dtype=torch.long)
    assert torch.equal(dec.generate(ids, 3, attention_mask=full, graph=False), dec.generate(ids, 3, graph=False))


@pytest.mark.parametrize("fused", [False, True])
def test_prefill_from_input_embeddings(fused):
    """prefill / generate with inputs_embeds (the VL case: image features in place of some token embeddings): with
    random vectors at some positions the last position's logits equal transformers' forward over the same embeddings,
    and the continuation equals transformers' greedy decoding of it; with the token embeddings themselves the result
    equals the ids-only request. Step-by-step prompt (eager steps) and the one-pass prefill."""
    net = tiny_lfm2(seed=12, conv_bias=True)
    lin = TorchLinears(decode_weights(net))
    B, T, H = 2, 7, net.config.hidden_size
    ids = torch.randint(3, net.config.vocab_size, (B, T), generator=torch.Generator().manual_seed(13))
    emb = net.model.embed_tokens(ids).detach().clone()
    emb[:, 2:5] = torch.randn(B, 3, H, generator=torch.Generator().manual_seed(14)) * 0.5  # "image" positions
    dec = StaticDecoder(net, bucket=16, keep_logits=True, fused_prefill=fused, linears=lin)
    first, st = dec.prefill(ids, 3, graph=False, inputs_embeds=emb)
    with torch.no_grad():
        want = net(inputs_embeds=emb, use_cache=False).logits.float()[:, -1]
    if fused:
        assert rel_err(dec.last_prefill_logits, want) < 1e-5
    else:
        assert rel_err(st.logits, want) < 1e-5
    want[:, dec.eos] = float("-inf")
    assert torch.equal(first, want.argmax(-1))
    out = dec.generate(ids, 3, graph=False, inputs_embeds=emb)
    with torch.no_grad():
        seq = emb
        for t in range(3):
            logits = net(inputs_embeds=seq, use_cache=False).logits.float()[:, -1]
            logits[:, dec.eos] = float("-inf")
            tok = logits.argmax(-1)
            assert torch.equal(out[:, T + t], tok), t
            seq = torch.cat([seq, net.model.embed_tokens(tok)[:, None]], dim=1)
    plain = net.model.embed_tokens(ids).detach()
    assert torch.equal(dec.generate(ids, 3, graph=False, inputs_embeds=plain), dec.generate(ids, 3, graph=False))
    with pytest.raises(ValueError, match="inputs_embeds must be"):
        dec.prefill(ids, 3, graph=False, inputs_embeds=emb[:, :-1])
    with pytest.raises(ValueError, match="LFM2-VL"):
        dec.prefill(ids, 3, graph=False, pixel_values=torch.zeros(1, 3, 8, 8))


def test_weight_keys_match_the_reference():
    """Keys and stacking order of the reference's StaticDecoder.lin (runtime.py:159-171, gptq.py:239-256)."""
    net = tiny_lfm2(seed=1, layer_types=("conv", "full_attention"))
    keys = decode_weight_modules(net)
    assert list(keys) == [("in", 0), ("out", 0), ("w13", 0), ("w2", 0), ("qkv", 1), ("o", 1), ("w13", 1), ("w2", 1),
                          ("head", 0)]
    assert keys[("qkv", 1)] == [f"model.layers.1.self_attn.{s}_proj" for s in "qkv"]
    assert keys[("w13", 0)] == ["model.layers.0.feed_forward.w1", "model.layers.0.feed_forward.w3"]
    w = decode_weights(net)
    a = net.model.layers[1].self_attn
    assert torch.equal(w[("qkv", 1)], torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]))
    f = net.model.layers[0].feed_forward
    assert torch.equal(w[("w13", 0)], torch.cat([f.w1.weight, f.w3.weight]))
    assert w[("head", 0)] is net.lm_head.weight


def test_decode_weight_file_round_trip(tmp_path):
    g = torch.Generator().manual_seed(2)
    pre = {("w13", 0): (torch.randint(0, 255, (64, 32), dtype=torch.uint8, generator=g), torch.rand(64, 1)),
           ("head", 0): (torch.randint(0, 255, (8, 32), dtype=torch.uint8, generator=g), torch.rand(8, 1),
                         torch.rand(64))}
    save_decode_weights(tmp_path / "w.pt", pre)
    back = load_decode_weights(tmp_path / "w.pt", device="cpu")
    assert set(back) == set(pre)
    for k in pre:
        assert all(torch.equal(a, b) for a, b in zip(back[k], pre[k]))
    torch.save({"w13": (torch.zeros(1),)}, tmp_path / "bad.pt")
    with pytest.raises(ValueError, match="not \\(kind, layer\\)"):
        load_decode_weights(tmp_path / "bad.pt", device="cpu")
    torch.save([torch.zeros(1)], tmp_path / "list.pt")
    with pytest.raises(ValueError, match="expected a dict"):
        load_decode_weights(tmp_path / "list.pt", device="cpu")


def expected_new_tokens(new, eos, n_new, check_every=4):
    """How many new tokens generate(stop_at_eos=True) returns for one row whose EOS-free greedy tokens are `new`:
    the prefill's token, then replays in chunks of 1, 2, 4, ... (at most check_every), stopping after the first
    chunk that leaves EOS among the tokens so far (runtime.py:473-492)."""
    if new[0] == eos:
        return 1
    n, done, chunk = n_new - 1, 0, 1
    while done < n:
        k = min(chunk, n - done)
        chunk = min(2 * chunk, check_every)
        done += k
        if done < n and eos in new[1:1 + done]:
            break
    return 1 + done


def test_generate_stop_at_eos():
    """stop_at_eos=True: EOS is not masked, and the replay loop stops at the first check (after 1, 2, 4, ... steps)
    where every row has produced it; the tokens are the EOS-free greedy run's (runtime.py:461-494). The linears are
    scaled up so that greedy decoding of the random model does not repeat one token, and EOS is the sixth new token:
    the checks after 1 and 3 replays miss it, the one after 7 sees it."""
    net = tiny_lfm2(seed=13, layer_types=("conv", "full_attention"))
    with torch.no_grad():
        for name, p in net.named_parameters():
            if name.endswith("proj.weight") or ".feed_forward.w" in name:
                p.mul_(4.0)
    dec = StaticDecoder(net, bucket=16, linears=TorchLinears(decode_weights(net)))
    dec.eos = dec.eos[:0]
    ids = torch.randint(3, net.config.vocab_size, (1, 5), generator=torch.Generator().manual_seed(3))
    free = dec.generate(ids, 12, graph=False)[0, 5:].tolist()  # no EOS token at all: plain greedy decoding
    assert free[5] not in free[:5], free
    dec.eos = torch.tensor([free[5]])
    out = dec.generate(ids, 12, stop_at_eos=True, graph=False)
    m = expected_new_tokens(free, free[5], 12)
    assert m == 8
    assert out.shape == (1, 5 + m) and out[0, 5:].tolist() == free[:m]
    # EOS as the very first token: no replay at all
    dec.eos = torch.tensor([free[0]])
    assert dec.generate(ids, 12, stop_at_eos=True, graph=False).shape == (1, 6)
