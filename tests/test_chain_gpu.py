"""The GEMV chain (lfm2q_gemv_chain: a decode step's GEMVs in one launch) against the same GEMVs run as separate
library calls, bit for bit, and against the CPU oracle on sampled rows.

The chains have real data dependencies -- an op reads what the op before it wrote (the residual stream h, the
SwiGLU activations, the attention-shaped outputs) -- so an op that started before its inputs were complete would
show up as a mismatch. Cases: a full LFM2-1.2B-shaped step (16 layers, 65 GEMVs, every epilogue) launched three
times in a row on one workspace (its launch counter advances), the exact op list the benchmark times, chains with
ops too small to give every workgroup a row and with uneven row splits and every supported K, and HIP-graph
replays. After each run the workspace's expired-wait word must be 0.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close_bf16, host_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import ext

    return ext()


def w8(g, N, K, gain=0.5):
    """int8 weights uniform over [-127, 127] with per-row scales (0.5 .. 1.5) gain / (73 sqrt(K)): an output row's
    magnitude is about gain times the input's RMS, so values stay finite through a step of dependent GEMVs
    (a uniform int8 weight has RMS 127 / sqrt(3) ~ 73)."""
    W = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    s = (torch.rand(N, device="cuda", generator=g) + 0.5) * (gain / (73.0 * K ** 0.5))
    return W, s


def same_bits(u, v):
    return torch.equal(u.contiguous().view(torch.int16), v.contiguous().view(torch.int16))


def run_separately(E, ops):
    for epi, W, s, x, y in ops:
        if epi == 0:
            E.gemv(W, s, x, y)
        elif epi == 1:
            E.gemv_epi(0, W, s, x, y)
        else:
            E.gemv_residual(W, s, x, y)


class Step:
    """Activation buffers of one dependent decode step: each GEMV reads what an earlier one wrote."""

    def __init__(self, g, layers, H=2048, FFN=8192, QKV=3072, CONV=6144, vocab=65536):
        bf = torch.bfloat16
        self.h = torch.randn(1, H, device="cuda", generator=g).to(bf)
        self.a = torch.empty(1, max(QKV, CONV), device="cuda", dtype=bf)  # qkv / in_proj outputs
        self.act = torch.empty(1, FFN, device="cuda", dtype=bf)
        self.logits = torch.empty(1, vocab, device="cuda", dtype=bf)

    def bufs(self):
        return [self.h, self.a, self.act, self.logits]


def step_ops(weights, st, types, H=2048, QKV=3072, CONV=6144):
    """Per layer: the attention / conv input projection reads h, the output projection reads the first H values
    of that projection and adds into h, w1|w3 reads h, w2 reads the SwiGLU activations and adds into h; the
    lm_head reads h."""
    ops, it = [], iter(weights)
    for t in types:
        Wi, si = next(it)
        n_in = QKV if t == "A" else CONV
        a_in = st.a[:, :n_in]
        ops.append((0, Wi, si, st.h, a_in))
        Wo, so = next(it)
        ops.append((2, Wo, so, st.a[:, :H], st.h))
        W13, s13 = next(it)
        ops.append((1, W13, s13, st.h, st.act))
        W2, s2 = next(it)
        ops.append((2, W2, s2, st.act, st.h))
    Wh, sh = next(it)
    ops.append((0, Wh, sh, st.h, st.logits))
    return ops


def make_weights(g, types, H=2048, FFN=8192, QKV=3072, CONV=6144, vocab=65536):
    ws = []
    for t in types:  # projections at gain 0.5, the layers that add into the residual stream at 0.1
        ws.append(w8(g, QKV if t == "A" else CONV, H))
        ws.append(w8(g, H, H, 0.1))
        ws.append(w8(g, 2 * FFN, H, 1.0))
        ws.append(w8(g, H, FFN, 0.1))
    ws.append(w8(g, vocab, H))
    return ws


def test_chain_full_decode_step_three_launches(E):
    """The 65-GEMV LFM2-1.2B step with dependencies through every op: three consecutive launches of one chain equal
    three rounds of the separate calls, bit for bit; one op's rows also against the oracle."""
    g = torch.Generator(device="cuda").manual_seed(21)
    types = "CCACCACCACACACAC"
    weights = make_weights(g, types)
    a = Step(g, len(types))
    b = Step(torch.Generator(device="cuda").manual_seed(22), len(types))
    b.h.copy_(a.h)
    ops_a, ops_b = step_ops(weights, a, types), step_ops(weights, b, types)
    chain = E.gemv_chain(ops_b)
    assert chain.n == 65
    for rep in range(3):
        run_separately(E, ops_a)
        chain()
        torch.cuda.synchronize()
        for u, v in zip(a.bufs(), b.bufs()):
            assert torch.isfinite(u.float()).all(), "test data overflowed"
            assert same_bits(u, v), f"launch {rep}: chain output differs from the separate calls"
        assert not chain.wait_expired()
    # the lm_head of the last launch against the oracle on 64 sampled rows
    Wh, sh = weights[-1]
    rows = torch.from_numpy(np.sort(np.random.default_rng(0).permutation(65536)[:64])).cuda()
    ref = oracle.gemv(Wh[rows].cpu().numpy(), sh[rows].cpu().numpy(), host_bits(b.h))
    assert_close_bf16(host_bits(b.logits)[:, rows.cpu().numpy()], ref, what="chain lm_head vs oracle")


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_chain_small_and_uneven_ops(E, seed):
    """Random chains over a residual stream h of width 1024 .. 8192: projections h -> t (plain or SwiGLU) with N
    from 1 row (most workgroups idle) through uneven splits (257, 1000, 3001 rows over the workgroups) to 8192, and
    residual ops t -> h that read the projection before them; every op depends on an earlier one."""
    r = np.random.default_rng(seed)
    g = torch.Generator(device="cuda").manual_seed(100 + seed)
    bf = torch.bfloat16
    Kh = int(r.choice([1024, 2048, 4096, 8192]))
    h_a = torch.randn(1, Kh, device="cuda", generator=g).to(bf)
    h_b = h_a.clone()
    ops_a, ops_b, outs = [], [], []
    t_a = t_b = None
    Kt = 0
    for _ in range(14):
        if t_a is not None and r.random() < 0.6:  # h += t W^T: reads the previous projection, writes h
            W, s = w8(g, Kh, Kt, 0.1)
            ops_a.append((2, W, s, t_a, h_a))
            ops_b.append((2, W, s, t_b, h_b))
            t_a = t_b = None
            continue
        epi = int(r.integers(0, 2))
        N = int(r.choice([1, 3, 100, 255, 256, 257, 1000, 1024, 2048, 3001, 4096, 8192]))
        W, s = w8(g, 2 * N if epi == 1 else N, Kh)
        ya = torch.empty(1, N, device="cuda", dtype=bf)
        yb = torch.empty(1, N, device="cuda", dtype=bf)
        ops_a.append((epi, W, s, h_a, ya))
        ops_b.append((epi, W, s, h_b, yb))
        outs.append((ya, yb))
        t_a, t_b, Kt = (ya, yb, N) if N in (1024, 2048, 4096, 8192) else (None, None, 0)
    chain = E.gemv_chain(ops_b)
    run_separately(E, ops_a)
    chain()
    torch.cuda.synchronize()
    assert torch.isfinite(h_a.float()).all(), "test data overflowed"
    for j, (u, v) in enumerate(outs):
        assert same_bits(u, v), f"projection {j}"
    assert same_bits(h_a, h_b), "residual stream"
    assert not chain.wait_expired()


def test_chain_graph_replays(E):
    """The chain captured into a HIP graph: every replay (with eager work and synchronizations between them) equals
    the separate calls repeated as often."""
    g = torch.Generator(device="cuda").manual_seed(5)
    types = "AC"
    weights = make_weights(g, types, vocab=8192)
    a = Step(g, 2, vocab=8192)
    b = Step(torch.Generator(device="cuda").manual_seed(6), 2, vocab=8192)
    b.h.copy_(a.h)
    ops_a, ops_b = step_ops(weights, a, types), step_ops(weights, b, types)
    chain = E.gemv_chain(ops_b)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    torch.cuda.synchronize()
    for rep in range(4):
        run_separately(E, ops_a)
        graph.replay()
        torch.cuda.synchronize()
        _ = (a.h.float() * 2).sum().item()  # unrelated eager work between replays
        for u, v in zip(a.bufs(), b.bufs()):
            assert same_bits(u, v), f"replay {rep}"
    assert not chain.wait_expired()


def test_chain_expired_wait_is_not_sticky(E, tune):
    """A launch whose dependency waits run out (forced from the host: a wait bound of 0 ms) reports it, and the next
    launch on the same workspace, with the normal bound, is not cut short by that error: its outputs equal the
    separate calls bit for bit and it reports no expired wait."""
    from lfm2opt import _capi

    g = torch.Generator(device="cuda").manual_seed(9)
    types = "AC"
    weights = make_weights(g, types, vocab=8192)
    a = Step(g, 2, vocab=8192)
    b = Step(torch.Generator(device="cuda").manual_seed(10), 2, vocab=8192)
    h0 = a.h.clone()
    b.h.copy_(h0)
    ops_a, ops_b = step_ops(weights, a, types), step_ops(weights, b, types)
    chain = E.gemv_chain(ops_b)
    tune("LFM2Q_CHAIN_WAIT_MS", 0)
    expired = False
    for _ in range(5):
        chain()
        torch.cuda.synchronize()
        if chain.wait_expired():
            expired = True
            break
    assert expired, "no wait ran out with a 0 ms bound"
    _capi.set_tuning("LFM2Q_CHAIN_WAIT_MS", None)
    b.h.copy_(h0)
    run_separately(E, ops_a)
    chain()
    torch.cuda.synchronize()
    assert not chain.wait_expired()
    for u, v in zip(a.bufs(), b.bufs()):
        assert same_bits(u, v), "the launch after an expired one differs from the separate calls"


def test_chain_argument_errors(E):
    W = torch.zeros(64, 1024, device="cuda", dtype=torch.int8)
    s = torch.ones(64, device="cuda")
    x = torch.zeros(1, 1024, device="cuda", dtype=torch.bfloat16)
    y = torch.zeros(1, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="at least one op"):
        E.gemv_chain([])
    with pytest.raises(RuntimeError, match="K must be 1024, 2048, 4096 or 8192"):
        E.gemv_chain([(0, W[:, :512].contiguous(), s, x[:, :512].contiguous(), y)])()
    with pytest.raises(RuntimeError, match="epi 0"):
        E.gemv_chain([(3, W, s, x, y)])
    with pytest.raises(RuntimeError, match=r"x \[1, K\]"):
        E.gemv_chain([(1, W[:63].contiguous(), s[:63].contiguous(), x, y)])
    with pytest.raises(RuntimeError, match="must be contiguous CUDA"):
        E.gemv_chain([(0, W, s.double(), x, y)])
    ops = [(0, W, s, x, y)] * 129
    with pytest.raises(RuntimeError, match="1 to 128 ops"):
        E.gemv_chain(ops)()
    torch.cuda.synchronize()
