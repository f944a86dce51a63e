"""lfm2q_gemv_chain_noalloc (the GEMV chain on the library's own per-GPU scratch array, no workspace argument)
against lfm2q_gemv_chain on its own workspace, called through the C ABI: bit for bit on every output, on calls in
a row whose sizes shrink and grow again (the scratch keeps the previous call's flags, so a stale flag would let an
op start early and show up as a mismatch), and under HIP-graph capture and replay. The status word must come back
0 every time."""

import ctypes

import pytest
import torch

from test_chain_gpu import Step, make_weights, same_bits, step_ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(cuda):
    from lfm2opt.kernels import ext

    return ext()


def noalloc(chain, status):
    """One lfm2q_gemv_chain_noalloc call on chain's op table (host and device copies)."""
    from lfm2opt import _capi

    _capi.call("lfm2q_gemv_chain_noalloc", ctypes.addressof(chain.host), chain.dev.data_ptr(), chain.n,
               status.data_ptr(), torch.cuda.current_stream().cuda_stream)


def pair(E, seed, types, vocab):
    """The same dependent decode step on two buffer sets: a through lfm2q_gemv_chain, b through the no-allocation
    entry point (b's table is only ever launched by noalloc)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    weights = make_weights(g, types, vocab=vocab)
    a = Step(g, len(types), vocab=vocab)
    b = Step(torch.Generator(device="cuda").manual_seed(seed + 1), len(types), vocab=vocab)
    b.h.copy_(a.h)
    return a, b, E.gemv_chain(step_ops(weights, a, types)), E.gemv_chain(step_ops(weights, b, types))


def check(a, b, what):
    for u, v in zip(a.bufs(), b.bufs()):
        assert torch.isfinite(u.float()).all(), "test data overflowed"
        assert same_bits(u, v), f"{what}: no-allocation chain differs from lfm2q_gemv_chain"


def test_noalloc_matches_chain_on_consecutive_calls(E):
    """Call 1: a 4-layer step (17 GEMVs, lm_head 16384 rows); call 2: a smaller 1-layer step (5 GEMVs, lm_head 2048
    rows); call 3: the first step again."""
    status = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    big = pair(E, 31, "CACA", 16384)
    small = pair(E, 41, "C", 2048)
    for k, (a, b, ca, cb) in enumerate([big, small, big]):
        print(f"noalloc call {k}: {cb.n} ops", flush=True)
        ca()
        status.fill_(7)
        noalloc(cb, status)
        torch.cuda.synchronize()
        check(a, b, f"call {k}")
        assert int(status.item()) == 0, f"call {k}: a dependency wait ran out"
        assert not ca.wait_expired()


def test_noalloc_graph_replays(E):
    """Captured into a HIP graph (the scratch clear is a kernel, so it replays), every replay with eager work
    between them equals lfm2q_gemv_chain repeated as often."""
    a, b, ca, cb = pair(E, 51, "AC", 8192)
    status = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    # one eager call first (as before any capture: the first call on a device looks up the scratch address)
    ca()
    noalloc(cb, status)
    torch.cuda.synchronize()
    check(a, b, "eager call before capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        noalloc(cb, status)
    torch.cuda.synchronize()
    for rep in range(4):
        print(f"noalloc replay {rep}", flush=True)
        ca()
        status.fill_(7)
        graph.replay()
        torch.cuda.synchronize()
        _ = (a.h.float() * 2).sum().item()  # unrelated eager work between replays
        check(a, b, f"replay {rep}")
        assert int(status.item()) == 0, f"replay {rep}: a dependency wait ran out"
