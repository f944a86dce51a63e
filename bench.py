#!/usr/bin/env python3
"""Benchmark of the quantized matmul hot path on one MI355X.

Headline workload: one LFM2-1.2B-shaped decode step run as weight-only INT8 GEMVs -- 16 layers typed
C C A C C A C C A C A C A C A C (6 attention, 10 short-conv), per attention layer qkv [3072x2048] and o [2048x2048]
(+residual), per conv layer in_proj [6144x2048] and out_proj [2048x2048] (+residual), per layer w1|w3 [16384x2048]
(+SwiGLU) and w2 [2048x8192] (+residual), then lm_head [65536x2048]. Every layer has its own weights (1.17 GB of
INT8 per step, so the 256 MB MALL cannot hold them). The 65 launches of one step are captured into a HIP graph;
a "step" is one replay. value = algorithmic bytes of the step / step time (GB/s), at batch 1; batches 4 and 16 are
reported alongside. Synthetic data: int8 weights uniform over [-127, 127], scales |N(0,1)| 0.01 + 1e-3, bf16
activations N(0, 1), seeded.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

import argparse
import ctypes
import json
import os
import pathlib
import platform
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "lfm2.5-vl-optimization_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

METRIC = "W8 GEMV HBM GB/s (% of peak) + W8A8 GEMM int8 TOPS (% MFMA) at LFM2 shapes"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
# HBM bytes per launch of the dominant decode kernel (w1|w3 16384 x 2048 INT8 + SwiGLU, batch 1), from two rocprofv3
# --pmc runs of `bench.py --eager-kind 'w1|w3+swiglu'` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled
# by what the counter reads for a 256 MiB device copy (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0): the run recorded in
# profiles/hbm_traffic_counters.md. Re-measure after changing that kernel.
W13_TRAFFIC_BYTES = 33947648
# W8A8 shapes (M, K, N, bias, gelu, name): LFM2 prefill at 512 / 2048 / 4096 tokens, SigLIP2 vision at 10 tiles
W8A8_SHAPES = ([(M, K, N, False, False, f"prefill M={M} {n}") for M in (512, 2048, 4096)
                for K, N, n in ((2048, 3072, "qkv"), (2048, 16384, "w1|w3"), (8192, 2048, "w2"))]
               + [(10240, 1152, 3456, True, False, "vision qkv"), (10240, 1152, 1152, True, False, "vision out"),
                  (10240, 1152, 4304, True, True, "vision fc1+gelu"), (10240, 4304, 1152, True, False, "vision fc2")])
LAYER_TYPES = "CCACCACCACACACAC"  # LFM2-1.2B layer order (A = attention, C = gated short conv)
H, FFN, VOCAB, QKV, CONV_IN = 2048, 8192, 65536, 3072, 6144


def gemv_bytes(N, K, B, residual=False):
    """Algorithmic bytes of one weight-only INT8 GEMV: W, scale, x and y once each (+ the residual read)."""
    return N * K + 4 * N + 2 * B * K + 2 * B * N + (2 * B * N if residual else 0)


def swiglu_bytes(S, K, B):
    return 2 * S * K + 4 * 2 * S + 2 * B * K + 2 * B * S


W4_GROUP = 128


def w4_bytes(N, K, B, residual=False, out=None):
    """Algorithmic bytes of one GPTQ-style INT4 GEMV over N weight rows: packed weights N K / 2, fp16 scales
    2 N K / 128, 4-bit zero points N K / 256, x, y (out columns; N unless SwiGLU) and the residual read."""
    out = N if out is None else out
    return N * K // 2 + 2 * N * K // W4_GROUP + N * K // (2 * W4_GROUP) + 2 * B * K + 2 * B * out \
        + (2 * B * out if residual else 0)


class DecodeStep:
    """All GEMVs of one decode step with distinct weights per layer, as a list of zero-argument launches.
    wfmt "int8": weight-only INT8 (per-row fp32 scales); "int4": GPTQ-style INT4 (int32 [N, K/8] packed weights,
    fp16 group scales |N(0,1)| 0.02 + 1e-3 and 4-bit zero points uniform over [0, 15], group 128)."""

    def __init__(self, B, device, seed=0, wfmt="int8"):
        from lfm2opt.kernels import ext

        E = ext()
        g = torch.Generator(device=device).manual_seed(seed)
        bf = torch.bfloat16

        def w8(N, K):
            W = torch.randint(-127, 128, (N, K), device=device, dtype=torch.int8, generator=g)
            s = torch.rand(N, device=device, generator=g) * 0.01 + 1e-3
            return W, s

        def w4(N, K):
            G = K // W4_GROUP
            qw = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), device=device, dtype=torch.int32, generator=g)
            sc = (torch.randn(N, G, device=device, generator=g).abs() * 0.02 + 1e-3).half()
            qz = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, (G + 7) // 8), device=device, dtype=torch.int32,
                               generator=g)
            return qw, sc, qz

        if wfmt == "int4":
            self._init_w4(E, B, device, g, w4)
            return

        self._dependent_buffers(B, device, g)
        self.ops = []        # (kind, fn, bytes)
        self.weights = []    # keep alive
        self.chain_ops = []  # the same GEMVs as (epi, W, scale, x, y) for the one-launch chain (batch 1)
        for t in LAYER_TYPES:
            if t == "A":
                Wq, sq = w8(QKV, H)
                Wo, so = w8(H, H)
                self.ops.append(("qkv", lambda W=Wq, s=sq: E.gemv(W, s, self.h, self.qkv), gemv_bytes(QKV, H, B)))
                self.ops.append(("o+res", lambda W=Wo, s=so: E.gemv_residual(W, s, self.mix, self.h),
                                 gemv_bytes(H, H, B, True)))
                self.chain_ops += [(0, Wq, sq, self.h, self.qkv), (2, Wo, so, self.mix, self.h)]
                self.weights += [Wq, sq, Wo, so]
            else:
                Wi, si = w8(CONV_IN, H)
                Wc, sc = w8(H, H)
                self.ops.append(("in", lambda W=Wi, s=si: E.gemv(W, s, self.h, self.bcx), gemv_bytes(CONV_IN, H, B)))
                self.ops.append(("out+res", lambda W=Wc, s=sc: E.gemv_residual(W, s, self.mix, self.h),
                                 gemv_bytes(H, H, B, True)))
                self.chain_ops += [(0, Wi, si, self.h, self.bcx), (2, Wc, sc, self.mix, self.h)]
                self.weights += [Wi, si, Wc, sc]
            W13, s13 = w8(2 * FFN, H)
            W2, s2 = w8(H, FFN)
            self.ops.append(("w1|w3+swiglu", lambda W=W13, s=s13: E.gemv_epi(0, W, s, self.h, self.act),
                             swiglu_bytes(FFN, H, B)))
            self.ops.append(("w2+res", lambda W=W2, s=s2: E.gemv_residual(W, s, self.act, self.h),
                             gemv_bytes(H, FFN, B, True)))
            self.chain_ops += [(1, W13, s13, self.h, self.act), (2, W2, s2, self.act, self.h)]
            self.weights += [W13, s13, W2, s2]
        Wh, sh = w8(VOCAB, H)
        self.ops.append(("lm_head", lambda: E.gemv(Wh, sh, self.h, self.logits), gemv_bytes(VOCAB, H, B)))
        self.chain_ops.append((0, Wh, sh, self.h, self.logits))
        self.weights += [Wh, sh]
        self.bytes = sum(b for _, _, b in self.ops)
        self.weight_bytes = sum(w.numel() * w.element_size() for w in self.weights if w.dtype == torch.int8)

    def _init_w4(self, E, B, device, g, w4):
        self._dependent_buffers(B, device, g)
        self.ops, self.weights = [], []

        def op(kind, N, K, x, y, epi, out=None):
            Wt = w4(N, K)
            self.weights += list(Wt)
            self.ops.append((kind, lambda Wt=Wt: E.gemv_w4z(*Wt, x, y, epi),
                             w4_bytes(N, K, B, residual=epi == 2, out=out)))

        for t in LAYER_TYPES:
            if t == "A":
                op("qkv", QKV, H, self.h, self.qkv, 0)
                op("o+res", H, H, self.mix, self.h, 2)
            else:
                op("in", CONV_IN, H, self.h, self.bcx, 0)
                op("out+res", H, H, self.mix, self.h, 2)
            op("w1|w3+swiglu", 2 * FFN, H, self.h, self.act, 1, out=FFN)
            op("w2+res", H, FFN, self.act, self.h, 2)
        op("lm_head", VOCAB, H, self.h, self.logits, 0)
        self.bytes = sum(b for _, _, b in self.ops)
        self.weight_bytes = sum(w.numel() * w.element_size() for w in self.weights)

    def _dependent_buffers(self, B, device, g):
        """Activations with the step's data dependencies: h is the residual stream (read by every projection,
        updated in place by o/out_proj and w2), the o/out_proj input is the first H values of the projection before
        it (at batch 1; the attention / short-conv between them is not part of this path), w2 reads the SwiGLU
        activations of w1|w3. The norms between are left out, so every GEMV reads what an earlier GEMV wrote."""
        bf = torch.bfloat16
        self.h = torch.randn(B, H, device=device, generator=g).to(bf)
        self.proj = torch.empty(B, max(QKV, CONV_IN), device=device, dtype=bf)  # qkv / in_proj output
        self.qkv, self.bcx = self.proj[:, :QKV], self.proj[:, :CONV_IN]
        if B == 1:
            self.mix = self.proj[:, :H]
        else:  # a column slice of several rows is not a contiguous GEMV input: its own buffer
            self.mix = torch.randn(B, H, device=device, generator=g).to(bf)
            self.qkv = torch.empty(B, QKV, device=device, dtype=bf)
            self.bcx = torch.empty(B, CONV_IN, device=device, dtype=bf)
        self.act = torch.empty(B, FFN, device=device, dtype=bf)
        self.logits = torch.empty(B, VOCAB, device=device, dtype=bf)

    def run(self, kinds=None):
        for kind, fn, _ in self.ops:
            if kinds is None or kind in kinds:
                fn()


_capture_stream = None


def capture(fn):
    """Capture fn's launches (all on torch's current stream) into a HIP graph. Warm-up and capture run on one stream
    kept for the process, so a library call that needs the stream's GEMM workspace creates it (and its zero fill)
    in the eager warm-up, never inside a graph."""
    global _capture_stream
    if _capture_stream is None:
        _capture_stream = torch.cuda.Stream()
    s = _capture_stream
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # eager warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        fn()
    torch.cuda.synchronize()
    return graph


def time_graph(graph, reps, warmup, warm_ms=0.0):
    """ms per replay over `reps` back-to-back replays, bracketed by synchronizations (HIP events on the stream),
    after `warmup` untimed replays and, with warm_ms, untimed replays for at least that long first (the matrix-core
    legs: clocks that dropped while the host prepared the next shape take ~0.1 s of load to come back)."""
    if warm_ms > 0:
        t_end = time.perf_counter() + warm_ms * 1e-3
        while time.perf_counter() < t_end:
            graph.replay()
            torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    t1.synchronize()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - w0) * 1e3 / reps
    return t0.elapsed_time(t1) / reps, wall


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(budget_s=10.0):
    """The reference's PyTorch dequant-matmul (tests/test_kernels.py:137, restated in oracle/cpu_baseline.py) over
    one decode step's worth of distinct GEMV shapes at batch 1, repeated until ~budget_s of CPU work."""
    from oracle.cpu_baseline import gemv_w8_dequant_matmul

    torch.set_num_threads(torch.get_num_threads())
    g = torch.Generator().manual_seed(0)
    shapes = [(QKV, H), (H, H), (CONV_IN, H), (2 * FFN, H), (H, FFN), (VOCAB, H)]
    mats = []
    for N, K in shapes:
        W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        s = torch.rand(N, generator=g) * 0.01 + 1e-3
        x = torch.randn(1, K, generator=g).to(torch.bfloat16)
        mats.append((W, s, x))
    nbytes = sum(gemv_bytes(N, K, 1) for N, K in shapes)
    for W, s, x in mats:  # warm-up
        gemv_w8_dequant_matmul(W, s, x)
    times, t_start = [], time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        for W, s, x in mats:
            gemv_w8_dequant_matmul(W, s, x)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"one each of the 6 decode GEMV shapes (qkv, o/out, in, w1|w3, w2, lm_head), batch 1, "
                      f"{nbytes / 1e6:.1f} MB per pass, median of {len(times)} passes; "
                      f"F.linear(x.float(), Wq.float() * scale[:, None]).to(bf16) with the dequant inside the "
                      f"timed region; os.cpu_count()={os.cpu_count()}, cpu='{cpu_model()}'"}


def _median_time(fn, budget_s, max_reps=50):
    fn()  # warm-up
    times, t_start = [], time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baselines_extra(budget_s=4.0):
    """The other CPU references of the path, each on a bounded sample (reported beside cpu_baseline, not used in
    `value`): the INT8 GEMV with the weights dequantized once outside the timed region, the INT4 GEMV (GPTQ-style,
    dequant inside, tests/test_kernels.py:150) and the W8A8 fake-quant GEMM (per-token quant + fp32 matmul of the
    dequantized operands, profiling/int8_quality_probe.py:150-160), all restated in oracle/cpu_baseline.py."""
    from oracle.cpu_baseline import gemv_w4_dequant_matmul, w8a8_fake_quant

    g = torch.Generator().manual_seed(1)
    cores = torch.get_num_threads()
    out = {}
    shapes = [(QKV, H), (H, H), (CONV_IN, H), (2 * FFN, H), (H, FFN), (VOCAB, H)]
    mats = []
    for N, K in shapes:
        W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        s = torch.rand(N, generator=g) * 0.01 + 1e-3
        mats.append((W.float() * s[:, None], torch.randn(1, K, generator=g).to(torch.bfloat16)))
    nbytes = sum(gemv_bytes(N, K, 1) for N, K in shapes)
    t, n = _median_time(lambda: [F.linear(x.float(), Wd).to(torch.bfloat16) for Wd, x in mats], budget_s)
    out["gemv_int8_dequantized_once"] = {
        "value": round(nbytes / t / 1e9, 3), "unit": "GB/s (INT8 algorithmic bytes)", "cores": cores, "kind": "port",
        "sample": f"the 6 decode GEMV shapes at batch 1, fp32 weights dequantized before timing, median of {n}"}
    w4 = []
    for N, K in shapes:
        G = K // W4_GROUP
        q = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
        z = torch.randint(0, 16, (N, G), generator=g, dtype=torch.uint8)
        sc = (torch.randn(N, G, generator=g).abs() * 0.02 + 1e-3).half()
        w4.append((q, sc, z, torch.randn(1, K, generator=g).to(torch.bfloat16)))
    nb4 = sum(w4_bytes(N, K, 1) for N, K in shapes)
    t, n = _median_time(lambda: [gemv_w4_dequant_matmul(q, sc, z, x, W4_GROUP) for q, sc, z, x in w4], budget_s)
    out["gemv_int4"] = {
        "value": round(nb4 / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": f"the 6 decode GEMV shapes at batch 1, GPTQ-style (group 128, zero points), dequant inside the "
                  f"timed region, {nb4 / 1e6:.1f} MB per pass, median of {n}"}
    M, K, N = 512, 2048, 3072
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 0.01 + 1e-3
    t, n = _median_time(lambda: w8a8_fake_quant(x, wq, sw), budget_s)
    out["w8a8_fake_quant"] = {
        "value": round(2.0 * M * N * K / t / 1e12, 4), "unit": "TOPS", "cores": cores, "kind": "port",
        "sample": f"prefill qkv {M}x{K}x{N}, per-token quant + fp32 matmul of the dequantized operands, median of {n}"}
    return out


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_results(B, steps, warmup, wfmt="int8"):
    log(f"decode step ({wfmt}), batch {B}: allocating weights")
    step = DecodeStep(B, "cuda", wfmt=wfmt)
    graph = capture(step.run)
    ms, wall = time_graph(graph, steps, warmup)
    res = {"batch": B, "ms_per_step": ms, "wall_ms_per_step": wall, "bytes_per_step": step.bytes,
           "gbs": step.bytes / ms / 1e6, "hbm_frac": step.bytes / ms / 1e6 / HBM_PEAK_GBS, "launches": len(step.ops)}
    # per-kind breakdown: each kind's launches alone, graph-captured, back to back
    kinds = {}
    for kind in dict.fromkeys(k for k, _, _ in step.ops):
        g = capture(lambda kind=kind: step.run({kind}))
        n = sum(1 for k, _, _ in step.ops if k == kind)
        kb = sum(b for k, _, b in step.ops if k == kind)
        kms, _ = time_graph(g, max(5, steps // 4), 3)
        kinds[kind] = {"launches": n, "us_per_launch": round(kms * 1e3 / n, 2), "gbs": round(kb / kms / 1e6, 1),
                       "bytes_per_launch": kb // n}
        del g
    res["kinds"] = kinds
    log(f"decode step ({wfmt}), batch {B}: {ms * 1e3:.1f} us/step, {res['gbs']:.0f} GB/s")
    if wfmt == "int8" and B == 1:
        res["chain"] = chain_results(step, steps, warmup)
        res["bandwidth_roof"] = bandwidth_roof(step)
    del graph, step
    torch.cuda.empty_cache()
    return res


def single_gemv_results(reps, cpu=True):
    """The standalone decode up-projection GEMV: x bf16 [1, 2048] ~ N(0, 1), W int8 [8192, 2048] uniform over
    [-127, 127], scale |N(0, 1)| 0.01 + 1e-3, y = bf16((x W^T) scale). Each call reads its own weights (>= 512 MB of
    distinct matrices rotated, as profiling/bench_gemv.py:40 does with 400 MB on its GPU), timed as graph replays
    and as eager back-to-back launches; beside it the reference's PyTorch dequant-matmul of the same GEMV
    (tests/test_kernels.py:137) on the host cores, on one matrix."""
    from lfm2opt.kernels import ext

    E = ext()
    N, K = 8192, 2048
    g = torch.Generator(device="cuda").manual_seed(0)
    ncopy = -(-512 * 2 ** 20 // (N * K))
    Ws = [torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g) for _ in range(ncopy)]
    ss = [torch.randn(N, device="cuda", generator=g).abs() * 0.01 + 1e-3 for _ in range(ncopy)]
    x = torch.randn(1, K, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty(1, N, device="cuda", dtype=torch.bfloat16)

    def run():
        for W, sc in zip(Ws, ss):
            E.gemv(W, sc, x, y)

    gr = capture(run)
    t_graph, _ = time_graph(gr, reps, 3)
    run()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(max(3, reps // 4)):
        run()
    t1.record()
    t1.synchronize()
    us_graph = t_graph * 1e3 / ncopy
    us_eager = t0.elapsed_time(t1) * 1e3 / (max(3, reps // 4) * ncopy)
    nbytes = gemv_bytes(N, K, 1)
    res = {"workload": "INT8 GEMV 8192 x 2048, batch 1", "bytes_per_call": nbytes, "weight_copies": ncopy,
           "us_graph": round(us_graph, 2), "gbs_graph": round(nbytes / us_graph / 1e3, 1),
           "hbm_frac_graph": round(nbytes / us_graph / 1e3 / HBM_PEAK_GBS, 4),
           "us_eager": round(us_eager, 2), "gbs_eager": round(nbytes / us_eager / 1e3, 1),
           "hbm_frac_eager": round(nbytes / us_eager / 1e3 / HBM_PEAK_GBS, 4)}
    del gr, Ws, ss
    torch.cuda.empty_cache()
    if cpu:
        from oracle.cpu_baseline import gemv_w8_dequant_matmul

        gc = torch.Generator().manual_seed(0)
        xc = torch.randn(1, K, generator=gc).to(torch.bfloat16)
        Wc = torch.randint(-127, 128, (N, K), generator=gc, dtype=torch.int8)
        sc = torch.randn(N, generator=gc).abs() * 0.01 + 1e-3
        t, n = _median_time(lambda: gemv_w8_dequant_matmul(Wc, sc, xc), 3.0)
        res["cpu_baseline"] = {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "us": round(t * 1e6, 1),
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"one 8192 x 2048 GEMV, F.linear(x.float(), Wq.float() * scale[:, None])"
                                         f".to(bf16) with the dequant inside the timed region, median of {n}"}
    return res


def chain_results(step, steps, warmup):
    """The same 65 GEMVs as one lfm2q_gemv_chain launch (each op waits on the device for the one before it, the
    weights of later ops streaming meanwhile), captured into a HIP graph of one node; a step is one replay."""
    from lfm2opt.kernels import ext

    chain = ext().gemv_chain(step.chain_ops)
    graph = capture(chain)
    ms, wall = time_graph(graph, steps, warmup)
    expired = chain.wait_expired()
    res = {"ms_per_step": ms, "wall_ms_per_step": wall, "bytes_per_step": step.bytes, "gbs": step.bytes / ms / 1e6,
           "hbm_frac": step.bytes / ms / 1e6 / HBM_PEAK_GBS, "launches": 1, "ops": chain.n, "wait_expired": expired}
    log(f"decode chain, batch 1: {ms * 1e3:.1f} us/step, {res['gbs']:.0f} GB/s" + (" WAIT EXPIRED" if expired else ""))
    del graph, chain
    return res


# Before each W8A8 timing: 150 ms of untimed replays, then W8A8_WARMUP more. After the host has spent a moment
# preparing a shape (or after 2 s idle) the first replays of a matrix-core-bound graph ran up to 18 % slower on
# MI355X (512 x 2048 x 16384: 26.3 -> 22.3 us over ~0.1 s of load, the same memory and graph), which left the
# first configuration timed per shape at a disadvantage. The HBM-bound decode step showed no such ramp (333.5 us
# cold and warm).
W8A8_WARMUP = 4
W8A8_WARM_MS = 150.0


def w8a8_results(reps):
    """Per shape: per-token quantization of the bf16 activations + W8A8 GEMM (bf16 out, bias / GELU where the
    layer has them), each call on its own weights (>= 512 MB of distinct weights rotated). Activations ~N(0,1)
    with 0.1% outliers at 20 sigma."""
    from lfm2opt import _capi
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    out = []
    for M, K, N, bias, gelu, name in W8A8_SHAPES:
        log(f"w8a8 {name} {M}x{K}x{N}")
        g = torch.Generator(device="cuda").manual_seed(M + K + N)
        ncopy = max(2, -(-512 * 2 ** 20 // (N * K)))
        Ws = [torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g) for _ in range(ncopy)]
        sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
        b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
        x = torch.randn(M, K, device="cuda", generator=g)
        x = torch.where(torch.rand(M, K, device="cuda", generator=g) < 1e-3, 20.0 * torch.sign(x), x)
        x = x.to(torch.bfloat16)
        xq = torch.empty(M, K, device="cuda", dtype=torch.int8)
        sx = torch.empty(M, device="cuda")
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)

        def full():
            for W in Ws:
                E.quant_rows(x, xq, sx)
                E.gemm_i8(xq, sx, W, sw, b, y, gelu)

        def gemm_only():
            for W in Ws:
                E.gemm_i8(xq, sx, W, sw, b, y, gelu)

        def int_mm():  # hipBLASLt's int8 GEMM with int32 output (no epilogue), the platform library's figure
            for W in Ws:
                torch._int_mm(xq, W.t())

        sx2 = torch.empty(M, device="cuda")

        def fused():  # the same pair as one call: row scales, then the GEMM quantizing x on its way into LDS
            for W in Ws:
                E.gemm_i8_bf16a(x, sx2, W, sw, b, y, gelu)

        xq3 = torch.empty(M, K, device="cuda", dtype=torch.int8)
        sx3 = torch.empty(M, device="cuda")

        def one_launch():  # the pair in one launch: the persistent GEMM quantizes x in its prologue
            for W in Ws:
                E.gemm_i8_fq(x, xq3, sx3, W, sw, b, y, gelu)

        g_full, g_gemm, g_lib, g_fused = capture(full), capture(gemm_only), capture(int_mm), capture(fused)
        _capi.set_tuning("LFM2Q_GEMM_FQ", 1)  # the one-launch kernel (the entry point's default is the pair)
        g_fq = capture(one_launch)
        _capi.set_tuning("LFM2Q_GEMM_FQ", None)
        t_full, _ = time_graph(g_full, reps, W8A8_WARMUP, W8A8_WARM_MS)
        t_gemm, _ = time_graph(g_gemm, reps, W8A8_WARMUP, W8A8_WARM_MS)
        t_lib, _ = time_graph(g_lib, reps, W8A8_WARMUP, W8A8_WARM_MS)
        t_fq, _ = time_graph(g_fq, reps, W8A8_WARMUP, W8A8_WARM_MS)
        t_fused, _ = time_graph(g_fused, max(3, reps // 4), 1)  # 3-6x slower than the pair: fewer replays
        us_full, us_gemm, us_lib = t_full * 1e3 / ncopy, t_gemm * 1e3 / ncopy, t_lib * 1e3 / ncopy
        us_fused, us_fq = t_fused * 1e3 / ncopy, t_fq * 1e3 / ncopy
        ops = 2.0 * M * N * K
        out.append({"name": name, "M": M, "K": K, "N": N, "bias": bias, "gelu": gelu,
                    "us_gemm": round(us_gemm, 2), "us_quant_gemm": round(us_full, 2),
                    "tops_gemm": round(ops / us_gemm / 1e6, 1), "tops_quant_gemm": round(ops / us_full / 1e6, 1),
                    "mfma_frac_gemm": round(ops / us_gemm / 1e6 / INT8_PEAK_TOPS, 4),
                    "us_hipblaslt_int_mm_i32": round(us_lib, 2), "tops_hipblaslt_int_mm_i32": round(ops / us_lib / 1e6, 1),
                    "us_fused_quant_gemm": round(us_fused, 2), "tops_fused_quant_gemm": round(ops / us_fused / 1e6, 1),
                    "us_one_launch_quant_gemm": round(us_fq, 2),
                    "tops_one_launch_quant_gemm": round(ops / us_fq / 1e6, 1)})
        del g_full, g_gemm, g_lib, g_fused, g_fq, Ws
        torch.cuda.empty_cache()
    return out


def eager_kind(kind, B, reps, wfmt="int8"):
    """Counter-collection mode: the launches of one decode kind (of the `wfmt` decode step), one W8A8 GEMM shape
    ("gemm:M,K,N", or "gemmg:M,K,N" with grouped-64 activation scales; gemm kernel only, on one weight matrix) or a
    plain 256 MiB device copy (kind "copy", the calibration of the HBM byte counters) run eagerly, one kernel per
    dispatch, `reps` times over."""
    if kind == "copy":
        src = torch.randint(-127, 128, (256 << 20,), device="cuda", dtype=torch.int8)
        dst = torch.empty_like(src)
        fns, nbytes = [lambda: dst.copy_(src)], 2 * src.numel()
    elif kind.startswith(("gemm:", "gemmg:")):
        from lfm2opt.kernels import int8_ext

        E8 = int8_ext()
        M, K, N = (int(v) for v in kind.split(":")[1].split(","))
        g = torch.Generator(device="cuda").manual_seed(M + K + N)
        w = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
        xq = torch.randint(-127, 128, (M, K), device="cuda", dtype=torch.int8, generator=g)
        sx, sw = torch.rand(M, device="cuda", generator=g), torch.rand(N, device="cuda", generator=g) * 0.01
        if kind.startswith("gemmg:"):  # grouped-64 activation scales [K/64, M]
            sx = torch.rand(K // 64, M, device="cuda", generator=g)
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        fns = [lambda: E8.gemm_i8(xq, sx, w, sw, None, y, False)]
        nbytes = M * K + N * K + 4 * sx.numel() + 4 * N + 2 * M * N
    else:
        step = DecodeStep(B, "cuda", wfmt=wfmt)
        sel = [(fn, b) for k, fn, b in step.ops if k == kind]
        if not sel:
            raise SystemExit(f"unknown kind {kind!r}: one of {sorted(set(k for k, _, _ in step.ops))} or copy")
        fns, nbytes = [fn for fn, _ in sel], sel[0][1]
    for fn in fns:
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        for fn in fns:
            fn()
    t1.record()
    t1.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / (reps * len(fns))
    print(json.dumps({"kind": kind, "wfmt": wfmt, "batch": B, "launches": reps * len(fns),
                      "us_per_launch_eager": round(us, 2), "bytes_per_launch": nbytes}))


def grouped_results(reps):
    """Grouped-64 W8A8 (grouped quant_rows + gemm_i8 with sxT [K/64, M]) and its INT8-output form gemm_i8_q, at the
    prefill / vision shapes whose K is a multiple of 64, each call on its own weights (>= 512 MB rotated)."""
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    out = []
    for M, K, N, bias, gelu, name in W8A8_SHAPES:
        if K % 64:
            continue
        g = torch.Generator(device="cuda").manual_seed(M + K + N + 1)
        ncopy = max(2, -(-512 * 2 ** 20 // (N * K)))
        Ws = [torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g) for _ in range(ncopy)]
        sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
        b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        xq = torch.empty(M, K, device="cuda", dtype=torch.int8)
        sxT = torch.empty(K // 64, M, device="cuda")
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        yq = torch.empty(M, N, device="cuda", dtype=torch.int8)
        ysT = torch.empty(N // 64, M, device="cuda") if N % 64 == 0 else None
        E.quant_rows(x, xq, sxT)
        g_gemm = capture(lambda: [E.gemm_i8(xq, sxT, W, sw, b, y, gelu) for W in Ws])
        t_gemm, _ = time_graph(g_gemm, reps, W8A8_WARMUP, W8A8_WARM_MS)
        ops = 2.0 * M * N * K
        r = {"name": name, "M": M, "K": K, "N": N, "us_gemm": round(t_gemm * 1e3 / ncopy, 2),
             "tops_gemm": round(ops / (t_gemm * 1e3 / ncopy) / 1e6, 1)}
        if ysT is not None:
            g_q = capture(lambda: [E.gemm_i8_q(xq, sxT, W, sw, b, yq, ysT, gelu) for W in Ws])
            t_q, _ = time_graph(g_q, reps, W8A8_WARMUP, W8A8_WARM_MS)
            r["us_gemm_i8_q"] = round(t_q * 1e3 / ncopy, 2)
            r["tops_gemm_i8_q"] = round(ops / (t_q * 1e3 / ncopy) / 1e6, 1)
            del g_q
        out.append(r)
        del g_gemm, Ws
        torch.cuda.empty_cache()
    return out


BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def lfm2_1p2b(device="cuda"):
    """transformers' Lfm2ForCausalLM with the LFM2-1.2B shapes (hidden 2048, 16 layers in LAYER_TYPES order, 32 query
    / 8 KV heads of 64, FFN 8192 after the config's 2/3 adjustment, vocab 65536, tied head), random weights, bf16."""
    from transformers import Lfm2Config, Lfm2ForCausalLM

    cfg = Lfm2Config(vocab_size=VOCAB, hidden_size=H, intermediate_size=12288, num_hidden_layers=len(LAYER_TYPES),
                     num_attention_heads=32, num_key_value_heads=8,
                     layer_types=["full_attention" if c == "A" else "conv" for c in LAYER_TYPES],
                     max_position_embeddings=128000, norm_eps=1e-5, conv_bias=False, tie_word_embeddings=True)
    torch.manual_seed(0)
    with torch.device(device):
        net = Lfm2ForCausalLM(cfg)
    return net.to(torch.bfloat16).eval()


def decode_e2e_results(steps, prompt=128, only=None):
    """Whole decode steps of LFM2-1.2B through lfm2opt.runtime.StaticDecoder: the library's linears and RMSNorms
    (add_rmsnorm_q) plus the PyTorch non-matmul ops (rotary embedding, attention over the static cache, short conv,
    argmax), one HIP graph per step, after a `prompt`-token prompt; random weights. "cublas" runs every linear
    through F.linear (hipBLASLt), the reference's baseline mode. only = "mode.batch" runs that one configuration."""
    from lfm2opt.runtime import StaticDecoder

    net = lfm2_1p2b()
    ids = torch.randint(3, VOCAB, (64, prompt), generator=torch.Generator().manual_seed(1)).cuda()
    out = {}
    for mode, batches in (("int8", (1, 8, 64)), ("int4", (1,)), ("bf16", (1,)), ("cublas", (1, 8, 64))):
        if only is not None:
            batches = [B for B in batches if f"{mode}.{B}" == only]
            if not batches:
                continue
        dec = StaticDecoder(net, gemv=mode)
        for B in batches:
            _, s = dec.prefill(ids[:B], steps + 1)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                s.graph.replay()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            out[f"{mode}.{B}"] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(B * 1e3 / ms, 1)}
            log(f"decode e2e {mode} batch {B}: {ms:.4f} ms per step")
        dec.clear_states()
        del dec, s
        torch.cuda.empty_cache()
    del net
    torch.cuda.empty_cache()
    return {"workload": f"LFM2-1.2B (random weights) greedy decode, prompt {prompt} tokens, {steps} timed steps, "
                        "cache bucket 256; whole step (linears + PyTorch non-matmul ops) as one HIP graph",
            "results": out}


def prefill_e2e_results(reps=5, only=None):
    """Whole-prompt prefill of LFM2-1.2B through lfm2opt.runtime (random weights, batch 1): "int8" = every GEMM but the
    head on W8A8 with the fused quantizing producers (prefill_int8; activation scales per 64-channel group, the
    default), "int8_per_token" = the same with one scale per token (LFM2_INT8_GROUP=0), "bf16" = the same pass on
    hipBLASLt BF16 GEMMs (fused_prefill in "cublas" mode); in all, the prompt's attention as bf16 batched products
    with an fp32 softmax. Median of `reps` eager passes. only: one configuration 'mode.tokens' (e.g. int8.2048)."""
    from lfm2opt.runtime import StaticDecoder

    tokens = (512, 2048)
    if only is not None and only not in {f"{n}.{T}" for n in ("int8", "int8_per_token", "bf16") for T in tokens}:
        raise ValueError(f"unknown prefill configuration {only!r}")
    net = lfm2_1p2b()
    out = {}
    for name, kw, group in (("int8", dict(gemv="int8", prefill_int8=True), None),
                            ("int8_per_token", dict(gemv="int8", prefill_int8=True), "0"),
                            ("bf16", dict(gemv="cublas", fused_prefill=True), None)):
        if only is not None and not only.startswith(name + "."):
            continue
        saved = os.environ.get("LFM2_INT8_GROUP")
        if group is not None:
            os.environ["LFM2_INT8_GROUP"] = group  # read when the W8A8 layers are built
        try:
            dec = StaticDecoder(net, **kw)
        finally:
            if group is not None:
                if saved is None:
                    os.environ.pop("LFM2_INT8_GROUP")
                else:
                    os.environ["LFM2_INT8_GROUP"] = saved
        for T in tokens:
            if only is not None and only != f"{name}.{T}":
                continue
            ids = torch.randint(3, VOCAB, (1, T), generator=torch.Generator().manual_seed(T)).cuda()
            s = dec.state(1, T + 1, 1, graph=False)
            times = []
            for r in range(reps + 1):
                s.clear()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                dec._prefill_batched(ids, s)
                e1.record()
                torch.cuda.synchronize()
                if r:
                    times.append(e0.elapsed_time(e1))
            ms = sorted(times)[len(times) // 2]
            out[f"{name}.{T}"] = {"ms": round(ms, 3), "tokens_per_s": round(T * 1e3 / ms, 1)}
            log(f"prefill e2e {name} {T} tokens: {ms:.3f} ms")
        del dec
        torch.cuda.empty_cache()
    del net
    torch.cuda.empty_cache()
    return {"workload": "LFM2-1.2B (random weights) prefill of one prompt of 512 / 2048 tokens in one pass "
                        "(16 layers + the head on the last position), eager", "results": out}


def w8a16_results(reps):
    """W8A16 gemm_w8 (the large-batch decode fallback and a vision layer), each call on its own weights."""
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    out = []
    for M, K, N, bias, gelu, name in ((64, 2048, 16384, False, False, "decode M=64 w1|w3"),
                                      (256, 2048, 16384, False, False, "decode M=256 w1|w3"),
                                      (256, 8192, 2048, False, False, "decode M=256 w2"),
                                      (10240, 1152, 4304, True, True, "vision fc1+gelu")):
        g = torch.Generator(device="cuda").manual_seed(M + K + N + 2)
        ncopy = max(2, -(-512 * 2 ** 20 // (N * K)))
        Ws = [torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g) for _ in range(ncopy)]
        sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
        b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        gr = capture(lambda: [E.gemm_w8(x, W, sw, b, y, gelu) for W in Ws])
        t, _ = time_graph(gr, reps, W8A8_WARMUP, W8A8_WARM_MS)
        us = t * 1e3 / ncopy
        nbytes = N * K + 2 * M * K + 2 * M * N + 4 * N
        out.append({"name": name, "M": M, "K": K, "N": N, "us": round(us, 2),
                    "tflops": round(2.0 * M * N * K / us / 1e6, 1), "gbs": round(nbytes / us / 1e3, 1)})
        del gr, Ws
        torch.cuda.empty_cache()
    return out


def producer_results(reps):
    """The activation quantizers and fused INT8 producers at prefill / vision shapes: algorithmic bytes (inputs and
    outputs once, at their dtypes) per call / time. Each op runs on rotating copies of its buffers (>= 512 MB in all,
    at least 4), all captured in one graph, so neither the graph launch nor a cache-resident input flatters or
    penalizes a single call."""
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    dev, bf = "cuda", torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(7)
    res = []

    def run(name, rows, L, make, nbytes):
        ncopy = max(4, -(-512 * 2 ** 20 // nbytes))
        fns = [make() for _ in range(ncopy)]
        gr = capture(lambda: [f() for f in fns])
        t, _ = time_graph(gr, reps, 2)
        us = t * 1e3 / ncopy
        res.append({"op": name, "rows": rows, "len": L, "us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1)})
        del gr, fns
        torch.cuda.empty_cache()

    def quant(rows, L, grouped):
        x = torch.randn(rows, L, device=dev, generator=g).to(bf)
        q = torch.empty(rows, L, device=dev, dtype=torch.int8)
        s = torch.empty((L // 64, rows) if grouped else (rows,), device=dev)
        return lambda: E.quant_rows(x, q, s)

    for rows, L, grouped in ((512, 8192, False), (4096, 2048, False), (4096, 2048, True), (10240, 1152, False),
                             (4096, 8192, True)):
        ns = (L // 64) * rows if grouped else rows
        run("quant_groups" if grouped else "quant_rows", rows, L, lambda: quant(rows, L, grouped),
            3 * rows * L + 4 * ns)

    def rmsnorm(rows, H, grouped):
        h = torch.randn(rows, H, device=dev, generator=g).to(bf)
        y = torch.randn(rows, H, device=dev, generator=g).to(bf)
        w = (torch.rand(H, device=dev, generator=g) + 0.5).to(bf)
        q = torch.empty(rows, H, device=dev, dtype=torch.int8)
        s = torch.empty((H // 64, rows) if grouped else (rows,), device=dev)
        return lambda: E.add_rmsnorm_q(h, y, w, q, s, 1e-5)

    for rows, H, grouped in ((4096, 2048, False), (4096, 2048, True)):
        ns = (H // 64) * rows if grouped else rows
        run(f"add_rmsnorm_q{' grouped' if grouped else ''}", rows, H, lambda: rmsnorm(rows, H, grouped),
            7 * rows * H + 2 * H + 4 * ns)

    def layernorm(rows, Dm):
        h = torch.randn(rows, Dm, device=dev, generator=g).to(bf)
        y = torch.randn(rows, Dm, device=dev, generator=g).to(bf)
        w = (torch.rand(Dm, device=dev, generator=g) + 0.5).to(bf)
        bb = torch.randn(Dm, device=dev, generator=g).to(bf)
        q = torch.empty(rows, Dm, device=dev, dtype=torch.int8)
        s = torch.empty(rows, device=dev)
        return lambda: E.add_layernorm_q(h, y, w, bb, q, s, 1e-6)

    run("add_layernorm_q", 10240, 1152, lambda: layernorm(10240, 1152), 7 * 10240 * 1152 + 4 * 1152 + 4 * 10240)

    def silu_q(rows, I):
        gg = torch.randn(rows, 2 * I, device=dev, generator=g).to(bf)
        q = torch.empty(rows, I, device=dev, dtype=torch.int8)
        s = torch.empty(rows, device=dev)
        return lambda: E.silu_mul_q(gg, q, s)

    run("silu_mul_q", 4096, 8192, lambda: silu_q(4096, 8192), 5 * 4096 * 8192 + 4 * 4096)
    return res


def quant_sweep(reps):
    """quant_rows / grouped quant_rows on the W8A8 workload's activation shapes under both launch forms (a wavefront
    per row, LFM2Q_QUANT_WG=0; a workgroup per row, =1) and the automatic choice, timed as producer_results times
    them (rotating copies, one graph): which form each shape should take."""
    from lfm2opt import _capi
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    dev, bf = "cuda", torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(3)
    res = []
    shapes = sorted({(M, K) for M, K, _, _, _, _ in W8A8_SHAPES})
    for M, K in shapes:
        for grouped in ((False, True) if K % 64 == 0 else (False,)):
            nbytes = 3 * M * K + 4 * ((K // 64) * M if grouped else M)
            ncopy = max(4, -(-512 * 2 ** 20 // nbytes))
            xs = [torch.randn(M, K, device=dev, generator=g).to(bf) for _ in range(ncopy)]
            qs = [torch.empty(M, K, device=dev, dtype=torch.int8) for _ in range(ncopy)]
            ss = [torch.empty((K // 64, M) if grouped else (M,), device=dev) for _ in range(ncopy)]
            row = {"rows": M, "len": K, "grouped": grouped}
            for name, val in (("wave", 0), ("wg", 1), ("auto", None)):
                _capi.set_tuning("LFM2Q_QUANT_WG", val)
                gr = capture(lambda: [E.quant_rows(x, q, sc) for x, q, sc in zip(xs, qs, ss)])
                t, _ = time_graph(gr, reps, 2)
                us = t * 1e3 / ncopy
                row[f"us_{name}"] = round(us, 2)
                row[f"gbs_{name}"] = round(nbytes / us / 1e3, 1)
                del gr
            _capi.set_tuning("LFM2Q_QUANT_WG", None)
            res.append(row)
            log(f"quant {M}x{K}{' grouped' if grouped else ''}: wave {row['us_wave']} us, wg {row['us_wg']} us, "
                f"auto {row['us_auto']} us")
            del xs, qs, ss
            torch.cuda.empty_cache()
    return res


def dispatch_sweep(reps, batches=(1, 4, 8, 16, 17, 24, 32, 48, 64, 96, 128, 256)):
    """The decode dispatch (lfm2opt/decode.py linear_path) against measurement: each decode weight shape at each batch
    on every path it could take -- the INT8 GEMV, W8A16 (with the K split), F.linear on the BF16 copy (hipBLASLt) and
    the GPTQ-style INT4 GEMV -- timed as one call per rotated weight copy in a graph (>= 512 MB of copies), with the
    path linear_path picks for INT8 and for INT4 weights (a BF16 copy kept) and how far each pick is from the
    fastest path available to that weight format."""
    from lfm2opt.decode import linear_path
    from lfm2opt.kernels import ext, int8_ext

    E, E8 = ext(), int8_ext()
    g = torch.Generator(device="cuda").manual_seed(4)
    shapes = [("qkv", QKV, H), ("in", CONV_IN, H), ("o", H, H), ("w13", 2 * FFN, H), ("w2", H, FFN),
              ("head", VOCAB, H)]
    res = []
    for name, N, K in shapes:
        nc = max(2, -(-512 * 2 ** 20 // (N * K * 2)))
        W8 = [torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g) for _ in range(nc)]
        Wb = [(torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16) for _ in range(nc)]
        W4 = [(torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), device="cuda", dtype=torch.int32, generator=g),
               (torch.rand(N, K // W4_GROUP, device="cuda", generator=g) * 0.02 + 1e-3).half(),
               torch.randint(-2 ** 31, 2 ** 31 - 1, (N, (K // W4_GROUP + 7) // 8), device="cuda", dtype=torch.int32,
                             generator=g)) for _ in range(nc)]
        s = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
        for B in batches:
            x = torch.randn(B, K, device="cuda", generator=g).to(torch.bfloat16)
            y = torch.empty(B, N, device="cuda", dtype=torch.bfloat16)
            t = {}
            for path, fn in (("gemv", lambda: [E.gemv(W, s, x, y) for W in W8]),
                             ("w8a16", lambda: [E8.gemm_w8(x, W, s, None, y, False) for W in W8]),
                             ("linear", lambda: [torch.mm(x, W.t(), out=y) for W in Wb]),
                             ("gemv_int4", lambda: [E.gemv_w4z(*W, x, y) for W in W4])):
                gr = capture(fn)
                t[path] = round(time_graph(gr, reps, 2)[0] * 1e3 / nc, 2)
                del gr
            p8 = linear_path("int8", "int8", B, N, K, True)
            p4 = linear_path("int4", "int4", B, N, K, True)
            best8 = min(("gemv", "w8a16", "linear"), key=t.get)
            best4 = min(("gemv_int4", "linear"), key=t.get)
            row = {"shape": name, "N": N, "K": K, "B": B, **{f"us_{k}": v for k, v in t.items()},
                   "pick_int8": p8, "best_int8": best8, "pick_int8_vs_best": round(t[p8] / t[best8], 3),
                   "pick_int4": p4, "best_int4": best4,
                   "pick_int4_vs_best": round(t["gemv_int4" if p4 == "gemv" else p4] / t[best4], 3)}
            res.append(row)
            log(f"dispatch {name} B={B}: " + ", ".join(f"{k} {v}" for k, v in t.items()) + f"; int8 pick {p8} "
                f"({row['pick_int8_vs_best']} x best), int4 pick {p4} ({row['pick_int4_vs_best']} x best)")
        del W8, Wb, W4
        torch.cuda.empty_cache()
    return res


# every (tile, K split) configuration of the per-token W8A8 kernels (the cost model's candidates); 256 x 256 and
# the first 256 x 128, 128 x 128 and 128 x 64 are the persistent kernels, "…/1g" the one-tile-per-workgroup kernels, "…sN"
# the persistent kernels with K cut into N slices over workgroups
GEMM_CONFIGS = [(256, 256, 1), (128, 256, 1), (128, 256, 2), (256, 128, 1), (256, 128, 1, 0), (256, 128, 2),
                (128, 128, 1), (128, 128, 1, 0), (128, 128, 2), (128, 64, 1), (128, 64, 2), (128, 64, 4), (64, 128, 1),
                (64, 128, 2), (64, 128, 4), (64, 64, 1), (64, 64, 2), (64, 64, 4), (256, 128, 1, 1, 2),
                (256, 128, 1, 1, 4), (128, 128, 1, 1, 2), (128, 128, 1, 1, 4), (128, 128, 1, 1, 8), (128, 64, 1, 0),
                (128, 64, 1, 1, 2), (128, 64, 1, 1, 4), (128, 64, 1, 1, 8), (256, 128, 1, 1, 8)]


def gemm_sweep(reps, only=None):
    """The per-token W8A8 GEMM on the 13 shapes under every forced (tile, K split) and under the automatic choice,
    timed as in w8a8_results (one call per rotated weight copy in a graph): how far the cost model's pick is from
    the best configuration of each shape."""
    from lfm2opt import _capi
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    knobs = ("LFM2Q_GEMM_BM", "LFM2Q_GEMM_BN", "LFM2Q_GEMM_KSPLIT", "LFM2Q_GEMM_BIGP", "LFM2Q_GEMM_SPLITK")
    out = []
    for M, K, N, bias, gelu, name in W8A8_SHAPES:
        if only and only not in name:
            continue
        log(f"sweep {name} {M}x{K}x{N}")
        g = torch.Generator(device="cuda").manual_seed(M + K + N)
        ncopy = max(2, -(-512 * 2 ** 20 // (N * K)))
        Ws = [torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g) for _ in range(ncopy)]
        sw = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-3
        b = torch.randn(N, device="cuda", generator=g).to(torch.bfloat16) if bias else None
        xq = torch.randint(-127, 128, (M, K), device="cuda", dtype=torch.int8, generator=g)
        sx = torch.rand(M, device="cuda", generator=g) * 0.01 + 1e-3
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)

        def fn():
            for W in Ws:
                E.gemm_i8(xq, sx, W, sw, b, y, gelu)

        us = {}
        try:
            for cfg in [None] + GEMM_CONFIGS:
                for k in knobs:
                    _capi.set_tuning(k, None)
                if cfg:
                    for k, v in zip(knobs, cfg):
                        _capi.set_tuning(k, v)
                graph = capture(fn)
                t = min(time_graph(graph, reps, W8A8_WARMUP, W8A8_WARM_MS)[0] for _ in range(2))
                label = "auto" if cfg is None else "%dx%d/%d" % cfg[:3] + (
                    "g" if len(cfg) == 4 else "s%d" % cfg[4] if len(cfg) > 4 else "")
                us[label] = round(t * 1e3 / ncopy, 2)
                del graph
        finally:
            for k in knobs:
                _capi.set_tuning(k, None)
        best = min((v, k) for k, v in us.items() if k != "auto")
        out.append({"name": name, "M": M, "K": K, "N": N, "us": us, "best": best[1], "us_best": best[0],
                    "us_auto": us["auto"]})
        del Ws
        torch.cuda.empty_cache()
    return {"shapes": out, "us_auto_total": round(sum(r["us_auto"] for r in out), 1),
            "us_best_total": round(sum(r["us_best"] for r in out), 1)}


_calib = None


def calib_lib():
    """lib/liblfm2q_calib.so: the calibration kernels (measurement equipment, not the product)."""
    global _calib
    if _calib is None:
        L = ctypes.CDLL(str(ROOT / "lfm2.5-vl-optimization_amd" / "lib" / "liblfm2q_calib.so"))
        L.lfm2q_calib_mfma_i8.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        L.lfm2q_calib_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_void_p]
        L.lfm2q_calib_fold_overlap.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_void_p]
        _calib = L
    return _calib


def stream_read(buf, nbytes, out, per_lane, aux=2):
    """One bare read of buf's first nbytes (calib stream_read_kernel) on torch's current stream."""
    st = calib_lib().lfm2q_calib_stream_read(buf.data_ptr(), nbytes, out.data_ptr(), per_lane, aux,
                                             torch.cuda.current_stream().cuda_stream)
    assert st == 0, st


def bandwidth_roof(step, reps=10):
    """The measured bandwidth roof of the decode GEMVs (the reference measured its practical DRAM roof with a 2 GB
    sum, docs/experiment_log.md:949). Kernels that only read (calib stream_read_kernel, 16-byte loads, 1-16 in
    flight per lane), replayed from HIP graphs:
      * `sizes`: one buffer of 4 MiB .. 1 GiB per launch, launches cycling over distinct buffers of at least 1 GiB in
        all (so no read comes from the 256 MB memory-side cache), best of the loads-per-lane settings, non-temporal
        loads (how the GEMVs read) and, at 1 GiB, cached loads too;
      * `step_graph`: one bare read per weight matrix of the INT8 decode step (the same 65 buffers, in step order,
        one launch each): what a graph of 65 kernels can reach with no arithmetic at all;
      * `node_floor_us`: a graph of 65 launches of one 16-byte read each: the per-node cost of a graph kernel.
    `measured_roof_gbs` is the best 1 GiB figure."""
    dev = "cuda"
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    MiB = 1 << 20
    pool = torch.empty(2048 * MiB, dtype=torch.uint8, device=dev)
    res = {"sizes": {}}
    for size_mib in (4, 16, 32, 128, 1024):
        nb = max(2, 1024 // size_mib)
        nbytes = size_mib * MiB
        bufs = [pool[i * nbytes:(i + 1) * nbytes] for i in range(nb)]
        row = {}
        for aux in ((2, 0) if size_mib == 1024 else (2,)):
            for per_lane in (1, 4, 8, 16):
                g = capture(lambda: [stream_read(b, nbytes, out, per_lane, aux) for b in bufs])
                ms, _ = time_graph(g, reps, 2)
                row[f"{'nt' if aux == 2 else 'cached'}_u{per_lane}"] = round(nbytes * nb / ms / 1e6, 1)
                del g
        best = max(row.values())
        res["sizes"][f"{size_mib}MiB"] = {"best_gbs": best, "us_per_launch": round(nbytes / best / 1e3, 2),
                                          "launches_per_graph": nb, **row}
        log(f"bare reads {size_mib} MiB: {best:.0f} GB/s")
    del pool
    torch.cuda.empty_cache()
    wts = [w for w in step.weights if w.dtype == torch.int8]
    wbytes = sum(w.numel() for w in wts)
    sg = {}
    for per_lane in (1, 8):
        g = capture(lambda: [stream_read(w, w.numel(), out, per_lane) for w in wts])
        ms, _ = time_graph(g, reps * 2, 3)
        sg[f"nt_u{per_lane}"] = {"us_per_step": round(ms * 1e3, 1), "gbs": round(wbytes / ms / 1e6, 1)}
        del g
    best = min(sg.values(), key=lambda r: r["us_per_step"])
    res["step_graph"] = {"launches": len(wts), "weight_bytes": wbytes, "best_us_per_step": best["us_per_step"],
                         "best_gbs": best["gbs"], **sg}
    log(f"bare reads of the decode step's 65 weight matrices: {best['us_per_step']} us, {best['gbs']:.0f} GB/s")
    g = capture(lambda: [stream_read(wts[0], 16, out, 1) for _ in wts])
    ms, _ = time_graph(g, reps * 4, 3)
    res["node_floor_us"] = round(ms * 1e3 / len(wts), 2)
    del g
    res["measured_roof_gbs"] = res["sizes"]["1024MiB"]["best_gbs"]
    return res


def read_branch_experiment(step, reps=40):
    """Staging the next weights through the memory-side cache on a concurrent branch, measured (the reference's
    programmatic dependent launch prefetches the next GEMV's weights before its dependency wait,
    kernels/lfm2_decode.cu:24-62): the INT8 batch-1 step's graph against the same graph with a second captured
    stream that reads weight matrix k (bare read kernel) once GEMV k - d has finished -- one cross-stream edge per
    GEMV, at most d matrices ahead -- and against a cached read of matrix i + 1 before each GEMV i on one stream."""
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    wts = [w for w in step.weights if w.dtype == torch.int8]
    fns = [fn for _, fn, _ in step.ops]
    res = {}

    def t(fn):
        g = capture(fn)
        ms, _ = time_graph(g, reps, 5)
        del g
        return round(ms * 1e3, 1)

    def branched(d, u, aux):
        main, side = torch.cuda.current_stream(), torch.cuda.Stream()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            for k in range(min(d, len(wts))):
                stream_read(wts[k], wts[k].numel(), out, u, aux)
        for i, fn in enumerate(fns):
            fn()
            if i + d < len(wts):
                ev = torch.cuda.Event()
                ev.record(main)
                side.wait_event(ev)
                with torch.cuda.stream(side):
                    stream_read(wts[i + d], wts[i + d].numel(), out, u, aux)
        main.wait_stream(side)

    def serial_next(u, aux):
        for i, fn in enumerate(fns):
            if i + 1 < len(wts):
                stream_read(wts[i + 1], wts[i + 1].numel(), out, u, aux)
            fn()

    res["step_us"] = t(step.run)
    for d in (1, 2, 3, 5):
        for u, aux in ((1, 0), (8, 0), (1, 2)):
            res[f"branch_d{d}_u{u}_{'cached' if aux == 0 else 'nt'}_us"] = t(lambda: branched(d, u, aux))
    res["serial_next_cached_us"] = t(lambda: serial_next(1, 0))
    res["reads_only_cached_us"] = t(lambda: [stream_read(w, w.numel(), out, 1, 0) for w in wts])
    log(f"read branch: step {res['step_us']} us, branched {min(v for k, v in res.items() if k.startswith('branch'))}"
        f" us at best, serial next-read {res['serial_next_cached_us']} us")
    return res


def mfma_rate(iters=20000):
    """The int8 matrix-core rate the chip sustains (lib/liblfm2q_calib.so: every SIMD issuing nothing but
    independent v_mfma_i32_32x32x32_i8, two wavefronts per SIMD) on random and on all-zero operand bytes, with the
    shader clock measured during the run (s_memtime against the 100 MHz s_memrealtime)."""
    L = calib_lib()
    blocks = 2 * torch.cuda.get_device_properties(0).multi_processor_count
    waves = 4 * blocks
    g = torch.Generator(device="cuda").manual_seed(7)
    srcs = {"random": torch.randint(-128, 128, (waves * 8 * 1024,), device="cuda", dtype=torch.int8, generator=g),
            "zeros": torch.zeros(waves * 8 * 1024, device="cuda", dtype=torch.int8)}
    out = torch.empty(waves * 64, device="cuda", dtype=torch.int32)
    clocks = torch.zeros(2, device="cuda", dtype=torch.int64)
    ops = waves * iters * 8 * 65536.0
    res = {}
    for name, src in srcs.items():
        def run():
            st = L.lfm2q_calib_mfma_i8(src.data_ptr(), src.numel(), out.data_ptr(), out.numel() * 4,
                                       clocks.data_ptr(), blocks, iters, torch.cuda.current_stream().cuda_stream)
            assert st == 0, st
        run()
        torch.cuda.synchronize()
        best = 1e30
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            run()
            e1.record()
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e-3)
        rt, sc = (int(v) for v in clocks.cpu())
        ghz = sc / rt * 0.1 if rt else None
        res[name] = {"tops": round(ops / best / 1e12, 1), "ms": round(best * 1e3, 3),
                     "clock_ghz": round(ghz, 3) if ghz else None,
                     "frac_of_published_peak": round(ops / best / 1e12 / INT8_PEAK_TOPS, 4)}
        log(f"mfma rate ({name} operands): {res[name]['tops']} TOPS at {res[name]['clock_ghz']} GHz")
    res["workload"] = f"{blocks} workgroups x 4 wavefronts x {iters} x 8 independent v_mfma_i32_32x32x32_i8"
    return res


def fq_overhead(reps=10):
    """The one-launch per-token W8A8 form (lfm2q_gemm_i8_fq with LFM2Q_GEMM_FQ=1) against its parts: quant_rows alone,
    the GEMM alone, the pair, and the one launch, at 512-10240 rows and N = 8 (one output tile: the time is the
    quantizing prologue, the wait for every chunk and the leaving count, beside a GEMM that is a few microseconds)
    and a full N; 20 calls per graph on one weight copy. Also the one launch with the steal bound at 0 (every waiting
    workgroup quantizes the chunks still open itself)."""
    from lfm2opt import _capi
    from lfm2opt.kernels import int8_ext

    E = int8_ext()
    out = []
    for M, K, N in ((64, 2048, 8), (512, 2048, 8), (512, 2048, 3072), (512, 8192, 2048), (4096, 8192, 8),
                    (4096, 8192, 2048), (10240, 4304, 1152)):
        g = torch.Generator(device="cuda").manual_seed(M + K + N)
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        W = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
        sw = torch.rand(N, device="cuda", generator=g) * 1e-3
        q = torch.empty(M, K, device="cuda", dtype=torch.int8)
        s = torch.empty(M, device="cuda")
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        R = 20

        def t(fn):
            gr = capture(lambda: [fn() for _ in range(R)])
            ms, _ = time_graph(gr, reps, W8A8_WARMUP, W8A8_WARM_MS)
            del gr
            return round(ms * 1e3 / R, 2)

        r = {"M": M, "K": K, "N": N, "us_quant": t(lambda: E.quant_rows(x, q, s)),
             "us_gemm": t(lambda: E.gemm_i8(q, s, W, sw, None, y, False))}
        r["us_pair"] = t(lambda: E.gemm_i8_fq(x, q, s, W, sw, None, y, False))  # the entry point's default
        try:
            _capi.set_tuning("LFM2Q_GEMM_FQ", 1)
            r["us_one_launch"] = t(lambda: E.gemm_i8_fq(x, q, s, W, sw, None, y, False))
            _capi.set_tuning("LFM2Q_GEMM_FQ_WAIT_US", 0)
            r["us_one_launch_steal_all"] = t(lambda: E.gemm_i8_fq(x, q, s, W, sw, None, y, False))
        finally:
            _capi.set_tuning("LFM2Q_GEMM_FQ", None)
            _capi.set_tuning("LFM2Q_GEMM_FQ_WAIT_US", None)
        r["one_launch_minus_gemm_us"] = round(r["us_one_launch"] - r["us_gemm"], 2)
        log(f"fq overhead {M}x{K}x{N}: {r}")
        out.append(r)
    return out


def fold_ceiling(iters=2000):
    """The grouped-64 fold's cost against the matrix work it folds (lib/liblfm2q_calib.so fold_overlap): per round of
    a 64 x 64 wavefront block, 8 v_mfma_i32_32x32x32_i8 alone, the fold's 64 conversions + 64 FMAs (+ 64 integer
    adds) alone, and both interleaved, at 1, 2 and 4 wavefronts per SIMD. Both ~= the vector work alone means the SIMD
    overlaps them and the fold's vector instructions, not the matrix core, bound the grouped GEMM."""
    L = calib_lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    inp = torch.randint(-100, 100, (512,), dtype=torch.int32, device="cuda")
    res = {}
    for per_simd in (1, 2, 4):
        blocks = cus * per_simd
        out = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
        row = {}
        for mode, name in ((0, "mfma_only"), (1, "fold_only"), (2, "both")):
            st = torch.cuda.current_stream().cuda_stream
            assert L.lfm2q_calib_fold_overlap(mode, inp.data_ptr(), out.data_ptr(), blocks, 20, st) == 0
            torch.cuda.synchronize()
            best = 1e30
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                assert L.lfm2q_calib_fold_overlap(mode, inp.data_ptr(), out.data_ptr(), blocks, iters, st) == 0
                e1.record()
                e1.synchronize()
                best = min(best, e0.elapsed_time(e1))
            row[name + "_ns_per_round"] = round(best * 1e6 / iters / per_simd, 1)
        row["both_over_fold_only"] = round(row["both_ns_per_round"] / row["fold_only_ns_per_round"], 3)
        row["both_over_sum"] = round(row["both_ns_per_round"] /
                                     (row["mfma_only_ns_per_round"] + row["fold_only_ns_per_round"]), 3)
        res[f"{per_simd}_waves_per_simd"] = row
        log(f"fold overlap, {per_simd} wave(s)/SIMD: {row}")
    res["workload"] = (f"{cus} x (1, 2, 4) workgroups of 4 wavefronts, {iters} rounds; ns per round per wavefront "
                       "(divided by the wavefronts sharing a SIMD)")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--batches", default="1,4,16", help="decode batch sizes to run (the first one is `value`)")
    ap.add_argument("--no-w8a8", action="store_true", help="skip the W8A8 GEMM shapes")
    ap.add_argument("--w4-batches", default="1,8", help="INT4 decode batch sizes ('' to skip)")
    ap.add_argument("--only-w8a8", action="store_true", help="W8A8 shapes only (no decode step, no CPU baseline)")
    ap.add_argument("--only-w8a16", action="store_true", help="W8A16 shapes only (no decode step, no CPU baseline)")
    ap.add_argument("--only-e2e", action="store_true",
                    help="only whole LFM2-1.2B decode steps through the decode runtime (lfm2opt.runtime)")
    ap.add_argument("--no-e2e", action="store_true", help="skip the whole-decode-step runtime leg")
    ap.add_argument("--e2e-mode", default=None,
                    help="with --only-e2e: one decode configuration 'mode.batch' (e.g. int8.1) and no prefill leg")
    ap.add_argument("--e2e-prompt", type=int, default=128,
                    help="with --only-e2e: prompt tokens before the timed decode steps (the cache grows with it)")
    ap.add_argument("--prefill-mode", default=None,
                    help="with --only-e2e: one prefill configuration 'mode.tokens' (e.g. int8.2048) and no decode leg")
    ap.add_argument("--only-w8a8-grouped", action="store_true",
                    help="grouped-64 W8A8 shapes only (no decode step, no CPU baseline)")
    ap.add_argument("--eager-kind", default=None,
                    help="run one decode kind (e.g. 'w1|w3+swiglu'), 'gemm:M,K,N', 'gemmg:M,K,N' (grouped scales) or 'copy' "
                         "eagerly, for counter collection")
    ap.add_argument("--wfmt", default="int8", choices=("int8", "int4"), help="decode weights for --eager-kind")
    ap.add_argument("--mfma-rate", action="store_true", help="only the sustained int8 matrix-core rate calibration")
    ap.add_argument("--bw-roof", action="store_true", help="only the bare-read bandwidth roof")
    ap.add_argument("--fq-overhead", action="store_true",
                    help="only the one-launch per-token W8A8 form against quant_rows, the GEMM and the pair")
    ap.add_argument("--fold-ceiling", action="store_true",
                    help="only the grouped fold's MFMA / vector-work overlap calibration")
    ap.add_argument("--dispatch-sweep", action="store_true",
                    help="only the decode linears on every path at batches 1-256 against the dispatch's pick")
    ap.add_argument("--quant-sweep", action="store_true",
                    help="only the activation quantizers under both launch forms on the W8A8 shapes")
    ap.add_argument("--read-branch", action="store_true",
                    help="only the decode step with a concurrent weight-read branch (memory-side-cache staging)")
    ap.add_argument("--sweep-only", default=None, help="--gemm-sweep: only the shapes whose name contains this")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="only the per-token W8A8 GEMM under every forced (tile, K split) on the 13 shapes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    if args.eager_kind:
        eager_kind(args.eager_kind, int(args.batches.split(",")[0]), args.steps, args.wfmt)
        return
    if args.gemm_sweep:
        print(json.dumps({"gemm_sweep": gemm_sweep(max(5, args.steps // 20), args.sweep_only)}))
        return
    if args.mfma_rate:
        print(json.dumps({"mfma_sustained": mfma_rate()}))
        return
    if args.fold_ceiling:
        print(json.dumps({"fold_ceiling": fold_ceiling()}))
        return
    if args.fq_overhead:
        print(json.dumps({"fq_overhead": fq_overhead()}))
        return
    if args.dispatch_sweep:
        print(json.dumps({"dispatch_sweep": dispatch_sweep(max(5, args.steps // 20))}))
        return
    if args.quant_sweep:
        print(json.dumps({"quant_sweep": quant_sweep(max(5, args.steps // 10))}))
        return
    if args.read_branch:
        print(json.dumps({"read_branch": read_branch_experiment(DecodeStep(1, "cuda"))}))
        return
    if args.bw_roof:
        step = DecodeStep(1, "cuda")
        print(json.dumps({"bandwidth_roof": bandwidth_roof(step, max(5, args.steps // 20))}))
        return
    if args.only_w8a8:
        print(json.dumps({"w8a8_shapes": w8a8_results(max(5, args.steps // 10))}))
        return
    if args.only_w8a16:
        print(json.dumps({"w8a16_shapes": w8a16_results(max(5, args.steps // 10))}))
        return
    if args.only_e2e:
        if args.e2e_mode:
            print(json.dumps({"decode_e2e": decode_e2e_results(max(16, args.steps // 4), prompt=args.e2e_prompt,
                                                               only=args.e2e_mode)}))
        elif args.prefill_mode:
            print(json.dumps({"prefill_e2e": prefill_e2e_results(only=args.prefill_mode)}))
        else:
            print(json.dumps({"decode_e2e": decode_e2e_results(max(16, args.steps // 4), prompt=args.e2e_prompt),
                              "prefill_e2e": prefill_e2e_results()}))
        return
    if args.only_w8a8_grouped:
        print(json.dumps({"w8a8_grouped": grouped_results(max(5, args.steps // 10))}))
        return
    batches = [int(b) for b in args.batches.split(",")]
    res1 = decode_results(batches[0], args.steps, args.warmup)
    extra = {B: decode_results(B, max(20, args.steps // 2), args.warmup) for B in batches[1:]}
    dom = res1["kinds"]["w1|w3+swiglu"]
    out = {
        "metric": METRIC,
        "value": round(res1["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "LFM2-1.2B decode step as weight-only INT8 GEMVs: 16 layers (6 attention, 10 "
                               "short-conv) + lm_head, 65 launches in one HIP graph, batch 1",
                   "batch": 1, "hidden": H, "ffn": FFN, "vocab": VOCAB, "bytes_per_step": res1["bytes_per_step"],
                   "compute": "int8 weights x bf16 activations, fp32 accumulation, bf16 out",
                   "parallelism": "single GPU"},
        "hbm_frac": round(res1["hbm_frac"], 4),
        "roofline": {"bound": "hbm", "kernel": "gemv_b1_kernel<int8,2,2,SWIGLU> (w1|w3 16384x2048 + SwiGLU)",
                     "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": W13_TRAFFIC_BYTES,
                     "us_per_launch": dom["us_per_launch"], "bytes_per_launch": dom["bytes_per_launch"]},
        "decode": {str(B): r for B, r in [(batches[0], res1)] + list(extra.items())},
    }
    roof = res1.get("bandwidth_roof")
    if roof:
        # the chip's measured streaming roof (bare 1 GiB reads) beside the 8 TB/s datasheet peak, and the step against
        # a graph of bare reads over its own 65 weight matrices
        out["roofline"]["measured_roof"] = roof["measured_roof_gbs"]
        out["roofline"]["frac_of_measured_roof"] = round(dom["gbs"] / roof["measured_roof_gbs"], 4)
        out["measured_roof_gbs"] = roof["measured_roof_gbs"]
        out["step_vs_bare_read_graph"] = round(roof["step_graph"]["best_us_per_step"] / (res1["ms_per_step"] * 1e3),
                                               4)
    log("single GEMV 8192 x 2048")
    out["single_gemv"] = single_gemv_results(max(20, args.steps // 2), cpu=not args.no_cpu)
    w4b = [int(b) for b in args.w4_batches.split(",") if b]
    if w4b:
        out["decode_w4"] = {str(B): decode_results(B, max(20, args.steps // 2), args.warmup, "int4") for B in w4b}
    if not args.no_e2e:
        log("decode e2e (runtime)")
        out["decode_e2e"] = decode_e2e_results(max(16, args.steps // 4))
        out["decode_e2e"]["gemv_only_step_ms_int8_b1"] = round(res1["ms_per_step"], 4)
        log("prefill e2e (runtime)")
        out["prefill_e2e"] = prefill_e2e_results()
    if not args.no_w8a8:
        shapes = w8a8_results(max(5, args.steps // 10))
        ops = sum(2.0 * r["M"] * r["N"] * r["K"] for r in shapes)
        t_gemm = sum(r["us_gemm"] for r in shapes)
        t_full = sum(r["us_quant_gemm"] for r in shapes)
        vis = [r for r in shapes if r["name"].startswith("vision")]
        vops = sum(2.0 * r["M"] * r["N"] * r["K"] for r in vis)
        t_lib = sum(r["us_hipblaslt_int_mm_i32"] for r in shapes)
        big = next(r for r in shapes if r["M"] == 4096 and r["N"] == 16384)
        out["w8a8"] = {"unit": "TOPS", "peak": INT8_PEAK_TOPS,
                       "roofline": {"bound": "mfma",
                                    "kernel": "gemm_i8_bigp_kernel<0, 256, 256, 2, false> (4096 x 2048 x 16384, persistent 256 x 256 tiles)",
                                    "achieved": big["tops_gemm"], "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                                    "frac": round(big["tops_gemm"] / INT8_PEAK_TOPS, 4)},
                       # the same layer as the workload specifies it: bf16 activations quantized per token
                       # (quant_rows) and then multiplied
                       "roofline_with_quant": {"bound": "mfma", "kernels": "quant_kernel + gemm_i8_bigp_kernel<0, 256, 256, 2, false>",
                                               "achieved": big["tops_quant_gemm"], "peak": INT8_PEAK_TOPS,
                                               "unit": "TOPS",
                                               "frac": round(big["tops_quant_gemm"] / INT8_PEAK_TOPS, 4)},
                       "mfma_sustained": mfma_rate(),
                       "all_shapes_tops_hipblaslt_int_mm_i32": round(ops / t_lib / 1e6, 1),
                       "all_shapes_tops_gemm": round(ops / t_gemm / 1e6, 1),
                       "all_shapes_tops_quant_gemm": round(ops / t_full / 1e6, 1),
                       "all_shapes_tops_fused_quant_gemm": round(ops / sum(r["us_fused_quant_gemm"] for r in shapes)
                                                                 / 1e6, 1),
                       "vision_layer_tops_gemm": round(vops / sum(r["us_gemm"] for r in vis) / 1e6, 1),
                       "vision_layer_tops_quant_gemm": round(vops / sum(r["us_quant_gemm"] for r in vis) / 1e6, 1),
                       "shapes": shapes}
    if not args.no_w8a8:
        log("grouped w8a8")
        out["w8a8_grouped"] = grouped_results(max(5, args.steps // 10))
        log("w8a16")
        out["w8a16"] = {"peak_tflops_bf16": BF16_PEAK_TFLOPS, "shapes": w8a16_results(max(5, args.steps // 10))}
        log("producers")
        out["producers"] = producer_results(max(10, args.steps // 5))
    if not args.no_cpu:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline()
        log("cpu baselines of the other paths")
        out["cpu_baselines_extra"] = cpu_baselines_extra()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
