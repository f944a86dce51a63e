"""Graph capture and stream concurrency of the library's entry points on the GPU.

Every entry point launches asynchronously on the caller's stream, allocates nothing and synchronizes nothing, so a
sequence of calls can be captured into a HIP graph. The test captures one of each kind of call (batch-1 / batch-2 /
matrix-core GEMVs with their epilogues, the INT4 GEMVs, the W8A8 GEMM with and without a K split, the grouped and
INT8-output GEMMs, W8A16, the quantizer and a fused producer), replays the graph several times with eager work,
synchronizations and new input values between the replays, and requires every replay to reproduce the eager results
bit for bit. A second test runs two independent call sequences on two streams at once and compares them with the
same sequences run one after the other.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ops(seed):
    """Operands and a closure that runs one of each call; returns (run, outputs, inputs)."""
    from lfm2opt.int8 import qbuf
    from lfm2opt.kernels import ext, int8_ext
    from lfm2opt.quant import quantize_int4_zp

    D, E8 = ext(), int8_ext()
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"
    w8 = torch.randint(-127, 128, (2048, 2048), device=dev, dtype=torch.int8, generator=g)
    s8 = torch.rand(2048, device=dev, generator=g) * 0.01 + 1e-3
    w4q, w4s, w4z = quantize_int4_zp((torch.randn(1024, 2048, device=dev, generator=g) * 0.02).to(torch.bfloat16))
    wq = torch.randint(-127, 128, (3072, 2048), device=dev, dtype=torch.int8, generator=g)
    sw = torch.rand(3072, device=dev, generator=g) * 0.01
    bias = torch.randn(3072, device=dev, generator=g).to(torch.bfloat16)
    inp = {
        "x1": torch.randn(1, 2048, device=dev, generator=g).to(torch.bfloat16),
        "x2": torch.randn(2, 2048, device=dev, generator=g).to(torch.bfloat16),
        "x8": torch.randn(8, 2048, device=dev, generator=g).to(torch.bfloat16),
        "xa": torch.randn(512, 2048, device=dev, generator=g).to(torch.bfloat16),
        "h": torch.randn(512, 2048, device=dev, generator=g).to(torch.bfloat16),
    }
    out = {
        "y1": torch.empty(1, 2048, device=dev, dtype=torch.bfloat16),
        "a1": torch.empty(1, 1024, device=dev, dtype=torch.bfloat16),
        "y2": torch.empty(2, 2048, device=dev, dtype=torch.bfloat16),
        "r8": torch.empty(8, 2048, device=dev, dtype=torch.bfloat16),
        "q1": torch.empty(1, 1024, device=dev, dtype=torch.bfloat16),
        "q8": torch.empty(8, 512, device=dev, dtype=torch.bfloat16),
        "xq": torch.empty(512, 2048, device=dev, dtype=torch.int8),
        "sx": torch.empty(512, device=dev, dtype=torch.float32),
        "g": torch.empty(512, 3072, device=dev, dtype=torch.bfloat16),
        "gs": torch.empty(64, 3072, device=dev, dtype=torch.bfloat16),
        "gq": torch.empty(512, 3072, device=dev, dtype=torch.bfloat16),
        "w8a16": torch.empty(512, 3072, device=dev, dtype=torch.bfloat16),
        "hn": torch.empty(512, 2048, device=dev, dtype=torch.bfloat16),
    }
    out["pq"], out["ps"] = qbuf(512, 2048, 64, dev)
    out["yq"], out["ys"] = qbuf(512, 3072, 64, dev)
    out["xg"], out["sg"] = qbuf(512, 2048, 64, dev)
    nw = torch.rand(2048, device=dev, generator=g).to(torch.bfloat16)
    hbase = torch.randn(8, 2048, device=dev, generator=g).to(torch.bfloat16)

    def run():
        D.gemv(w8, s8, inp["x1"], out["y1"])                       # batch 1
        D.gemv_epi(0, w8, s8, inp["x1"], out["a1"])                # batch 1 + SwiGLU
        D.gemv(w8, s8, inp["x2"], out["y2"])                       # batch 2 (VALU)
        out["r8"].copy_(hbase)
        D.gemv_residual(w8, s8, inp["x8"], out["r8"])              # batch 8 (matrix cores) + residual
        D.gemv_w4z(w4q, w4s, w4z, inp["x1"], out["q1"])            # INT4 batch 1
        D.gemv_w4z(w4q, w4s, w4z, inp["x8"], out["q8"], epi=1)     # INT4 batch 8 + SwiGLU
        E8.quant_rows(inp["xa"], out["xq"], out["sx"])             # per-token quantizer
        E8.gemm_i8(out["xq"], out["sx"], wq, sw, bias, out["g"], True)        # W8A8 (+ bias, GELU)
        E8.gemm_i8(out["xq"][:64], out["sx"][:64], wq, sw, None, out["gs"], False)  # 64 tokens: K split
        E8.quant_rows(inp["xa"], out["xg"], out["sg"])             # grouped-64 quantizer
        E8.gemm_i8(out["xg"], out["sg"], wq, sw, bias, out["gq"], False)      # grouped W8A8
        E8.gemm_i8_q(out["xg"], out["sg"], wq, sw, None, out["yq"], out["ys"], False)  # INT8 output
        E8.gemm_w8(inp["xa"], wq, sw, bias, out["w8a16"], False)   # W8A16
        E8.add_rmsnorm_q(inp["h"], inp["xa"], nw, out["pq"], out["ps"], 1e-5, out["hn"])  # fused producer

    return run, out, inp


def _snapshot(out):
    return {k: v.clone() for k, v in out.items()}


def test_graph_replays_match_eager(cuda):
    from lfm2opt.kernels import prepare_workspace

    run, out, inp = _ops(1)
    h0 = inp["h"].clone()
    run()  # warm-up outside the capture (library load, first-call setup)
    cap = torch.cuda.Stream()
    prepare_workspace(stream=cap)  # the capture stream's GEMM workspace, zero-filled outside the graph
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        run()
    g = torch.Generator(device="cuda").manual_seed(7)
    for rep in range(3):
        # new input values between replays: the graph must read the live buffers
        for k in ("x1", "x2", "x8", "xa"):
            inp[k].copy_(torch.randn(inp[k].shape, device="cuda", generator=g).to(torch.bfloat16))
        inp["h"].copy_(h0)
        torch.cuda.synchronize()
        run()
        torch.cuda.synchronize()
        eager = _snapshot(out)
        inp["h"].copy_(h0)
        for v in out.values():
            v.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, v in out.items():
            assert torch.equal(v, eager[k]), f"replay {rep}: {k} differs from the eager call"


def test_two_streams_match_serial(cuda):
    runs = [_ops(11), _ops(12)]
    h0 = [inp["h"].clone() for _, _, inp in runs]
    for (run, _, _) in runs:
        run()
    torch.cuda.synchronize()
    serial = [_snapshot(out) for _, out, _ in runs]
    for (run, out, inp), h in zip(runs, h0):
        inp["h"].copy_(h)
        for v in out.values():
            v.fill_(0)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for (run, _, _), s in zip(runs, streams):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            run()
    torch.cuda.synchronize()
    for i, (_, out, _) in enumerate(runs):
        for k, v in out.items():
            assert torch.equal(v, serial[i][k]), f"stream {i}: {k} differs from the serial run"


def test_capture_without_workspace_raises(cuda):
    """A GEMM that needs its stream's workspace inside a capture, before the workspace exists, raises: the zero fill
    would otherwise exist only in that graph and leave the K-split counters undefined for the next user."""
    from lfm2opt.kernels import int8_ext, release_workspace

    E8 = int8_ext()
    xq = torch.ones(64, 2048, device="cuda", dtype=torch.int8)
    sx = torch.ones(64, device="cuda")
    wq = torch.ones(3072, 2048, device="cuda", dtype=torch.int8)
    sw = torch.ones(3072, device="cuda")
    y = torch.empty(64, 3072, device="cuda", dtype=torch.bfloat16)
    cap = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="prepare_workspace"):
        with torch.cuda.graph(graph, stream=cap):
            E8.gemm_i8(xq, sx, wq, sw, None, y, False)
    torch.cuda.synchronize()
    assert not release_workspace(stream=cap)  # nothing was created for it


def test_two_graphs_on_one_capture_stream(cuda):
    """Two graphs captured on one stream share its workspace: replaying the second one first, then the first, then
    eager calls on that stream all reproduce the eager results, K split included (64 tokens: 24 tiles)."""
    from lfm2opt.kernels import int8_ext, prepare_workspace, release_workspace

    E8 = int8_ext()
    g = torch.Generator(device="cuda").manual_seed(5)
    wq = torch.randint(-127, 128, (3072, 2048), device="cuda", dtype=torch.int8, generator=g)
    sw = torch.rand(3072, device="cuda", generator=g) * 0.01
    xs = [torch.randn(64, 2048, device="cuda", generator=g).to(torch.bfloat16) for _ in range(2)]
    qs = [(torch.empty(64, 2048, device="cuda", dtype=torch.int8), torch.empty(64, device="cuda")) for _ in xs]
    ys = [torch.empty(64, 3072, device="cuda", dtype=torch.bfloat16) for _ in xs]

    def call(i):
        E8.quant_rows(xs[i], *qs[i])
        E8.gemm_i8(qs[i][0], qs[i][1], wq, sw, None, ys[i], False)

    for i in range(2):
        call(i)
    torch.cuda.synchronize()
    eager = [y.clone() for y in ys]
    cap = torch.cuda.Stream()
    prepare_workspace(stream=cap)
    torch.cuda.synchronize()
    graphs = [torch.cuda.CUDAGraph() for _ in range(2)]
    for i in range(2):
        with torch.cuda.graph(graphs[i], stream=cap):
            call(i)
    for rep in range(3):
        for y in ys:
            y.fill_(0)
        torch.cuda.synchronize()
        graphs[1].replay()
        graphs[0].replay()
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(ys[i], eager[i]), f"rep {rep}: graph {i} differs from the eager call"
        with torch.cuda.stream(cap):
            for i in range(2):
                call(i)
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(ys[i], eager[i]), f"rep {rep}: eager call {i} on the capture stream differs"
    del graphs
    torch.cuda.synchronize()
    assert release_workspace(stream=cap)
