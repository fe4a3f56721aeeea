"""Benchmark of the block-scaled FP8 path on one MI355X.

Headline workload: the decode-shape dense FP8 linear sweep -- bf16
activations ``[M, 2048]`` (~N(0,1), 1% of entries x20) for M in
{1, 4, 16, 64, 256} against e4m3 weights ``[6144, 2048]`` with 128x128 f32
block scales; one step = one ``fp8_linear`` (1x128 quantize + block-scaled
MFMA GEMM, bf16 out) per M.  The value is whole-step algorithmic HBM bytes
per second, ``sum_M N*K + 4*ceil(N/128)*K/128 + 2*M*K + 2*M*N`` over the
step time.  Every op of a step reads its own copy of the weights, from a
rotation of more than twice the 256 MB last-level cache, which is emptied
before the timed region, so weights stream from HBM.  ``--warmup W`` steps
run first, then exactly ``--steps K`` steps are timed as one replay of a HIP
graph holding them.

Also reported: ``roofline`` for the dominant op of the step (the M=256
``fp8_linear``, every launch it makes), ``roofline_prefill`` for the
prefill ``fp8_linear`` op at M=8192, K=2048, N=6144 (its quantizer and GEMM
launches; MFMA-bound), ``ceilings`` measured by the probe library
(streaming HBM read, FP8 MFMA), ``extras`` (the single M=16, K=N=2048 linear
the reference's CPU path runs, the prefill GEMMs, the MoE decode layer
unpacked and packed, the skewed MoE prefill layer, the fused RMSNorm + quantizer
and the shared-expert MoE block; each MoE block timed as one of four
captured back to back in a graph, as a decode step graph holds many layers)
and ``cpu_baseline`` (the oracle's C restatement on the host cores, per
config).

    python bench.py [--steps K] [--warmup W] [--no-extras] [--no-cpu]
    python bench.py --kernel-probe {decode,decode_m1,decode_m4,decode_m16,decode_m64,
                                    prefill,moe_decode,moe_prefill,copy}
                                  # launches for rocprofv3 --pmc passes
    python bench.py --roofline-probe   # the measured ceilings alone
    python bench.py --operand-probe    # prefill GEMM: random against constant operands
    python bench.py --library-ab LIB [LIB ...]   # prefill GEMMs, library builds interleaved
    python bench.py --vendor-probe     # prefill GEMM beside hipBLASLt's FP8 GEMMs
"""

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "FP8 GEMM/MoE TFLOPS and HBM GB/s vs roofline at M=1..16384, 1 MI355X"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
DECODE_M = (1, 4, 16, 64, 256)
K_DEC, N_DEC = 2048, 6144


def dense_bytes(m, k, n, scale_bytes=4):
    return n * k + scale_bytes * math.ceil(n / 128) * (k // 128) + 2 * m * k + 2 * m * n


def gemm_kernel_bytes(m, k, n):
    """Algorithmic bytes of the GEMM launch alone: weights + block scales,
    prequantized codes + scales in, bf16 out."""
    return n * k + 4 * math.ceil(n / 128) * (k // 128) + m * k + 4 * m * (k // 128) + 2 * m * n


def make_weights(torch, n, k, copies, seed, dev):
    """``copies`` independent e4m3 weight sets, N(0, 0.02) block-quantized on the GPU."""
    from akas_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    codes, scales = [], []
    for _ in range(copies):
        w = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32) * 0.02
        c, s = ops.quantize_weight_blocks(w)
        codes.append(c)
        scales.append(s)
        del w
    return codes, scales


def bf16_activations(torch, m, k, seed, dev, outliers=0.01):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    if outliers:
        mask = rng.random((m, k)) < outliers
        x = np.where(mask, x * np.float32(20), x).astype(np.float32)
    return torch.from_numpy(x).to(dev).to(torch.bfloat16)


_SLEEP_PER_MS = None


def _hold_gpu(torch, ms):
    """Enqueue a GPU-side spin of about ``ms`` milliseconds so that the launches
    queued behind it are timed back to back, free of host dispatch gaps."""
    global _SLEEP_PER_MS
    if _SLEEP_PER_MS is None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        a.record()
        torch.cuda._sleep(1_000_000)
        b.record()
        torch.cuda.synchronize()
        _SLEEP_PER_MS = 1_000_000 / max(a.elapsed_time(b), 1e-3)
    torch.cuda._sleep(int(_SLEEP_PER_MS * ms))


def time_kernel(torch, fn, reps, hold_ms=None):
    """Average GPU duration of the launch(es) made by ``fn(i)``: a start/end
    event pair on the current stream around each call, all enqueued behind a
    GPU spin so the events see GPU time only."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    torch.cuda.synchronize()
    _hold_gpu(torch, hold_ms if hold_ms is not None else 0.06 * reps + 2)
    for i in range(reps):
        starts[i].record()
        fn(i)
        ends[i].record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / reps  # ms


def time_kernel_graph(torch, fn, n, replays=5):
    """Average GPU duration per launch of ``fn(i)``, from a HIP graph of ``n``
    back-to-back launches timed with one event pair per replay (no per-launch
    event packets, no host dispatch gaps)."""
    g = graph_of(torch, fn, n)
    g.replay()
    a = [torch.cuda.Event(enable_timing=True) for _ in range(replays)]
    b = [torch.cuda.Event(enable_timing=True) for _ in range(replays)]
    torch.cuda.synchronize()
    for i in range(replays):
        a[i].record()
        g.replay()
        b[i].record()
    torch.cuda.synchronize()
    return min(x.elapsed_time(y) for x, y in zip(a, b)) / n  # ms, best replay


def graph_of(torch, fn, n):
    """HIP graph of ``fn(0) .. fn(n-1)`` on a side stream (warmed up first)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    return g


LLC_BYTES = 256 << 20  # MI355X last-level cache (MALL)


def _evict_llc(torch, dev):
    """Write 1 GiB (four times the last-level cache) so that no weight copy
    is cache-resident when a timed region starts."""
    buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    torch.cuda.synchronize()
    del buf


def decode_sweep(torch, dev, steps, warmup):
    """The headline: ``warmup`` eager steps, then exactly ``steps`` steps timed
    as one replay of a graph that holds them, with a barrier (synchronize) on
    both sides.  Every op reads its own weight copy: op j of step i reads copy
    (5 i + j) mod ``copies``, and the copies hold more than twice the
    last-level cache, so no launch reads a copy that the previous
    ``copies - 1`` launches left in the cache; the cache is emptied before the
    timed replay, so its first launches read cold copies too."""
    from akas_amd import ops

    wbytes = N_DEC * K_DEC
    copies = math.ceil(2 * LLC_BYTES / wbytes) + 1
    codes, scales = make_weights(torch, N_DEC, K_DEC, copies, 1234, dev)
    xs = {m: bf16_activations(torch, m, K_DEC, m, dev) for m in DECODE_M}
    outs = {m: torch.empty((m, N_DEC), dtype=torch.bfloat16, device=dev) for m in DECODE_M}
    ws = ops.linear_workspace(max(DECODE_M), K_DEC, N_DEC, dev)
    step_bytes = sum(dense_bytes(m, K_DEC, N_DEC) for m in DECODE_M)

    def step(i):
        for j, m in enumerate(DECODE_M):
            c = (len(DECODE_M) * i + j) % copies
            ops.fp8_linear(xs[m], codes[c], scales[c], out=outs[m], workspace=ws)

    for i in range(warmup):
        step(i)
    g = graph_of(torch, step, steps)
    g.replay()  # the graph's first replay uploads it; untimed
    torch.cuda.synchronize()
    _evict_llc(torch, dev)
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    del g

    # Per M: the fp8_linear op as the step runs it (every launch it makes),
    # and the GEMM launch alone on prequantized codes; each averaged over a
    # graph of `copies` back-to-back launches on the launching stream.
    per_m = []
    for m in DECODE_M:
        op_ms = time_kernel_graph(torch, lambda i: ops.fp8_linear(
            xs[m], codes[i % copies], scales[i % copies], out=outs[m], workspace=ws), copies)
        q, qs = ops.quantize(xs[m])
        ms = time_kernel_graph(torch, lambda i: ops.projection_partial(
            q, qs, codes[i % copies], scales[i % copies], out=outs[m],
            out_dtype=torch.bfloat16), copies)
        ob, b = dense_bytes(m, K_DEC, N_DEC), gemm_kernel_bytes(m, K_DEC, N_DEC)
        per_m.append(dict(M=m, op_us=round(op_ms * 1e3, 3), op_bytes=ob,
                          op_gbs=round(ob / (op_ms * 1e-3) / 1e9, 1),
                          op_frac_hbm=round(ob / (op_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                          gemm_us=round(ms * 1e3, 3), gemm_bytes=b,
                          gemm_gbs=round(b / (ms * 1e-3) / 1e9, 1),
                          tflops=round(2 * m * K_DEC * N_DEC / (op_ms * 1e-3) / 1e12, 2)))
    return dict(step_s=dt, step_bytes=step_bytes, per_m=per_m, copies=copies, steps=steps,
                touched=min(copies, len(DECODE_M) * steps))


PREFILL_SHAPES = ((2048, 6144), (2048, 8192), (8192, 2048))


def prefill_gemms(torch, dev, steps):
    """Config 3: M=8192, fused activation quantize, bf16 out.  ``op``: the
    fp8_linear call (all its launches); ``gemm``: its GEMM launch alone, on
    prequantized codes (the same kernel); ``gemm_bf16_scales``: that launch
    with the weight scales in bf16."""
    from akas_amd import ops

    res = []
    for (k, n) in PREFILL_SHAPES:
        m = 8192
        codes, scales = make_weights(torch, n, k, 1, 7 + n, dev)
        x = bf16_activations(torch, m, k, 99, dev, outliers=0.0)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        ws = ops.linear_workspace(m, k, n, dev)
        fn = lambda i: ops.fp8_linear(x, codes[0], scales[0], out=out, workspace=ws)
        for i in range(3):
            fn(i)
        ms_total = time_kernel(torch, fn, steps)
        q, qs = ops.quantize(x)
        ms_gemm = time_kernel(torch, lambda i: ops.projection_partial(
            q, qs, codes[0], scales[0], out=out, out_dtype=torch.bfloat16), steps)
        flops = 2 * m * k * n
        # the same GEMM with bf16 weight scales (the block-FP8 checkpoints' dtype)
        scales_bf16 = scales[0].to(torch.bfloat16)
        ms_bf16 = time_kernel(torch, lambda i: ops.projection_partial(
            q, qs, codes[0], scales_bf16, out=out, out_dtype=torch.bfloat16), steps)
        res.append(dict(M=m, K=k, N=n, op_us=round(ms_total * 1e3, 2),
                        gemm_us=round(ms_gemm * 1e3, 2), gemm_bf16_scales_us=round(ms_bf16 * 1e3, 2),
                        op_tflops=round(flops / (ms_total * 1e-3) / 1e12, 1),
                        gemm_tflops=round(flops / (ms_gemm * 1e-3) / 1e12, 1),
                        op_frac_fp8=round(flops / (ms_total * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                        gemm_frac_fp8=round(flops / (ms_gemm * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4)))
        del codes, scales, x, out
    return res


LAYERS_PER_GRAPH = 4  # MoE blocks captured back to back in one graph


def moe_layer_bench(torch, dev, tokens, zipf, steps, packed=False):
    """The routed MoE block (router, routes, grouped gate/up with SwiGLU and
    re-quantize, grouped down, combine).  packed: the reference's packed
    policy (an expert_pack copy, then contiguous expert rows); unpacked, the
    grouped kernels gather each expert's rows through the route table
    themselves, with bit-identical outputs."""
    from akas_amd import moe

    H, F, E, top = 2048, 1536, 64, 4
    bank = {}
    for name, (n, k) in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
        c, s = make_weights(torch, n, k, E, {"w1": 1, "w3": 3, "w2": 2}[name], dev)
        bank[name] = (torch.stack(c), torch.stack(s))
        del c, s
    wts = moe.ExpertWeights(*bank["w1"], *bank["w3"], *bank["w2"])
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.normal(0, 1, (tokens, H)).astype(np.float32)).to(dev).to(torch.bfloat16)
    logits = rng.normal(0, 1, (tokens, E)).astype(np.float32)
    if zipf:
        logits += (-1.1 * np.log1p(rng.permutation(E))).astype(np.float32)[None, :]
    logits = torch.from_numpy(logits).to(dev)
    fn = lambda i: moe.routed_moe(x, logits, None, wts, top=top, packed=packed,
                                  max_block_m=128 if packed else 64,
                                  product_dtype=torch.bfloat16, activation_dtype=torch.bfloat16,
                                  contribution_dtype=torch.bfloat16)
    # Several layers per graph, as a decode program captures a whole step:
    # the per-replay graph launch is shared by LAYERS_PER_GRAPH layers.
    g = graph_of(torch, fn, LAYERS_PER_GRAPH)
    g.replay()
    ms = time_kernel(torch, lambda i: g.replay(), steps) / LAYERS_PER_GRAPH
    _, routing = moe.routed_moe(x, logits, None, wts, top=top, return_routing=True)
    counts = routing["counts"].cpu().numpy()
    active_experts = int((counts > 0).sum())
    flops = 6 * F * H * tokens * top
    wbytes = active_experts * 3 * F * H
    abytes = 2 * tokens * H + tokens * H + tokens * top * (H + F) + tokens * top * H * 2 + 2 * tokens * H
    del bank, wts
    return dict(T=tokens, zipf=zipf, packed=packed, us=round(ms * 1e3, 2),
                tflops=round(flops / (ms * 1e-3) / 1e12, 1),
                gbs=round((wbytes + abytes) / (ms * 1e-3) / 1e9, 1),
                frac_hbm=round((wbytes + abytes) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                frac_fp8=round(flops / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                max_expert_rows=int(counts.max()), mean_expert_rows=float(counts.mean()))


def shared_expert_block_bench(torch, dev, tokens=64, steps=10):
    """The Qwen3.5 block-fp8 MoE block at decode: 256 experts, top 8,
    H=2048, F=512, plus the sigmoid-gated shared expert."""
    from akas_amd import moe

    H, F, E, top = 2048, 512, 256, 8
    bank = {}
    for name, (n, k), copies in (("w1", (F, H), E), ("w3", (F, H), E), ("w2", (H, F), E),
                                 ("sw1", (F, H), 1), ("sw3", (F, H), 1), ("sw2", (H, F), 1)):
        c, s = make_weights(torch, n, k, copies, 11, dev)
        bank[name] = (torch.stack(c), torch.stack(s)) if copies > 1 else (c[0], s[0])
    wts = moe.ExpertWeights(*bank["w1"], *bank["w3"], *bank["w2"])
    shared = moe.SharedExpert(*bank["sw1"], *bank["sw3"], *bank["sw2"])
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.normal(0, 1, (tokens, H)).astype(np.float32)).to(dev).to(torch.bfloat16)
    logits = torch.from_numpy(rng.normal(0, 1, (tokens, E)).astype(np.float32)).to(dev)
    gate = torch.from_numpy(rng.normal(0, 1, tokens).astype(np.float32)).to(dev)
    fn = lambda i: moe.shared_expert_moe(x, logits, gate, wts, shared, top=top)
    g = graph_of(torch, fn, LAYERS_PER_GRAPH)
    g.replay()
    ms = time_kernel(torch, lambda i: g.replay(), steps) / LAYERS_PER_GRAPH
    ids = torch.topk(logits.to(torch.bfloat16).float(), top, dim=1).indices
    active_experts = int(torch.unique(ids).numel())
    wbytes = (active_experts + 1) * 3 * F * H
    del bank, wts, shared
    return dict(T=tokens, experts=E, top=top, us=round(ms * 1e3, 2),
                gbs=round(wbytes / (ms * 1e-3) / 1e9, 1),
                frac_hbm=round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                active_experts=active_experts)


def config1_linear_bench(torch, dev, m=16, k=2048, n=2048):
    """The single linear the reference's CPU path runs (M=16, K=N=2048, bf16
    in and out, f32 block scales): one ``fp8_linear`` op per launch, each on
    its own weight copy from a rotation of more than twice the last-level
    cache, so the weights stream from HBM as in the decode sweep."""
    from akas_amd import ops

    copies = math.ceil(2 * LLC_BYTES / (n * k)) + 1
    codes, scales = make_weights(torch, n, k, copies, 4321, dev)
    x = bf16_activations(torch, m, k, 7, dev)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    ws = ops.linear_workspace(m, k, n, dev)
    us = time_kernel_graph(torch, lambda i: ops.fp8_linear(
        x, codes[i % copies], scales[i % copies], out=out, workspace=ws), copies) * 1e3
    nbytes = dense_bytes(m, k, n)
    del codes, scales
    return dict(M=m, K=k, N=n, us=round(us, 3), bytes=nbytes,
                gbs=round(nbytes / (us * 1e-6) / 1e9, 1),
                frac_hbm=round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                tflops=round(2 * m * n * k / (us * 1e-6) / 1e12, 2))


def rms_quantize_bench(torch, dev, rows=16384, cols=2048, steps=20):
    """RMSNorm fused with the quantizer (the producer of the MoE block's and
    the projections' FP8 input): bf16 x in, bf16 normalized rows + codes +
    scales out, rotating over enough row blocks to stream from HBM."""
    from akas_amd import ops

    copies = 8  # 8 x (64 + 64 + 32) MB in rotation, past the 256 MB MALL
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    xs = [torch.randn((rows, cols), generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
    w = torch.rand((cols,), generator=g, device=dev) + 0.5
    ys = [torch.empty((rows, cols), dtype=torch.bfloat16, device=dev) for _ in range(copies)]
    cs = [torch.empty((rows, cols), dtype=torch.uint8, device=dev) for _ in range(copies)]
    ss = [torch.empty((rows, cols // 128), dtype=torch.float32, device=dev) for _ in range(copies)]
    fn = lambda i: ops.rms_quantize(xs[i % copies], w, eps=1e-5, normalized=ys[i % copies],
                                    out=cs[i % copies], scales=ss[i % copies])
    us = time_kernel_graph(torch, fn, copies) * 1e3
    nbytes = rows * cols * (2 + 2 + 1) + rows * (cols // 128) * 4 + cols * 4
    del xs, ys, cs, ss
    return dict(rows=rows, cols=cols, us=round(us, 2), gbs=round(nbytes / (us * 1e-6) / 1e9, 1),
                frac_hbm=round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))


def _cpu_model():
    """The host CPU's model name from /proc/cpuinfo (None where absent)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _median_time(fn, runs, budget_s):
    """Median wall time of ``fn()`` after one warm-up run: at least ``runs``
    runs, more while ``budget_s`` lasts (at most 50)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < runs or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def _random_codes(rng, shape):
    """Finite e4m3 codes (magnitude code <= 126, either sign): the CPU path's
    time does not depend on the values."""
    n = int(np.prod(shape))
    return (np.frombuffer(rng.bytes(n), np.uint8) & np.uint8(0xFE)).reshape(shape)


def cpu_baseline():
    """The oracle's C restatement (oracle/cpu_ref.c, -O3 -fopenmp, f32
    accumulation, LUT weight decode) timed on the host cores with
    ``os.cpu_count()`` threads, per config: the decode sweep in full (the
    headline's baseline, also on one thread as the reference's CI runs its
    CPU checks), config 1 in full, bounded row/token samples of configs 3
    and 5, and the MoE decode layer of config 4 in full."""
    from oracle import native
    from oracle import fp8 as ofp8

    lib = native.load()
    threads = os.cpu_count() or 1
    p = native.ptr
    rng = np.random.default_rng(0)
    per = {}

    def linear_case(m, k, n, label, sample, runs=5, budget=3.0):
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        codes, scales = ofp8.quantize_weight_blocks(w)
        x = ofp8.bf16_bits(rng.normal(0, 1, (m, k)).astype(np.float32))
        out = np.empty((m, n), np.uint16)
        t, count = _median_time(lambda: lib.ref_fp8_linear_bf16(
            p(x), p(codes), p(scales), p(out), 1, m, k, n, threads), runs, budget)
        b = dense_bytes(m, k, n)
        per[label] = dict(ms=round(t * 1e3, 3), gbs=round(b / t / 1e9, 3),
                          gflops=round(2 * m * k * n / t / 1e9, 2), runs=count, sample=sample)

    linear_case(16, 2048, 2048, "config1_linear_m16", "full: x [16, 2048], W [2048, 2048]")
    linear_case(256, 2048, 6144, "config3_prefill_gemm",
                "256 of the 8192 rows of M=8192, K=2048, N=6144 (rate scales with rows)")

    # config 2, the headline's baseline: the full sweep
    w = rng.normal(0, 0.02, (N_DEC, K_DEC)).astype(np.float32)
    codes, scales = ofp8.quantize_weight_blocks(w)
    xs = {m: ofp8.bf16_bits(rng.normal(0, 1, (m, K_DEC)).astype(np.float32)) for m in DECODE_M}
    outs = {m: np.empty((m, N_DEC), np.uint16) for m in DECODE_M}

    def sweep(nthreads):
        for m in DECODE_M:
            lib.ref_fp8_linear_bf16(p(xs[m]), p(codes), p(scales), p(outs[m]), 1, m, K_DEC, N_DEC,
                                    nthreads)

    med, runs = _median_time(lambda: sweep(threads), 5, 8.0)
    med1, runs1 = _median_time(lambda: sweep(1), 5, 0.0)
    step_bytes = sum(dense_bytes(m, K_DEC, N_DEC) for m in DECODE_M)

    # configs 4 and 5: the MoE layer (H=2048, F=1536, 64 experts, top 4)
    H, F, E, top = 2048, 1536, 64, 4
    w1, w3, w2 = (_random_codes(rng, sh) for sh in ((E, F, H), (E, F, H), (E, H, F)))
    s13 = rng.uniform(2e-4, 1e-3, (E, F // 128, H // 128)).astype(np.float32)
    s2 = rng.uniform(2e-4, 1e-3, (E, H // 128, F // 128)).astype(np.float32)

    def moe_case(tokens, zipf, label, sample, runs):
        x = ofp8.bf16_bits(rng.normal(0, 1, (tokens, H)).astype(np.float32))
        logits = rng.normal(0, 1, (tokens, E)).astype(np.float32)
        if zipf:
            logits += (-1.1 * np.log1p(rng.permutation(E))).astype(np.float32)[None, :]
        out = np.empty((tokens, H), np.float32)
        t, count = _median_time(lambda: lib.ref_moe_layer_bf16(
            p(x), p(logits), p(w1), p(s13), p(w3), p(s13), p(w2), p(s2), p(out), tokens, H, F, E,
            top, threads), runs, 0.0)
        flops = 6 * F * H * tokens * top
        per[label] = dict(ms=round(t * 1e3, 2), gflops=round(flops / t / 1e9, 2), runs=count,
                          sample=sample)

    moe_case(256, False, "config4_moe_decode", "full: T=256, all 64 experts active", 5)
    moe_case(512, True, "config5_moe_prefill_zipf",
             "512 of the 16384 tokens, same Zipf(1.1) logit offsets (rate scales with tokens)", 5)
    return dict(value=round(step_bytes / med / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                cpu_model=_cpu_model(), host_cpus=os.cpu_count(),
                sample=f"full decode sweep (M=1,4,16,64,256; K=2048; N=6144), median of {runs} "
                       f"runs, {med * 1e3:.1f} ms/sweep, oracle/cpu_ref.c -O3 -fopenmp, f32 "
                       f"accumulation",
                value_1_thread=round(step_bytes / med1 / 1e9, 3),
                sample_1_thread=f"same sweep on 1 thread, median of {runs1} runs, "
                                f"{med1 * 1e3:.1f} ms/sweep",
                per_config=per)


def profile_value(name, key):
    """``key: value`` from a committed profile summary under profiles/, or
    None when the summary or the key is absent."""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return float(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


DECODE_COUNTERS = "decode_fp8_linear_m256_counters.md"
PREFILL_COUNTERS = "prefill_gemm_counters.md"
PROBE_M = 256          # the sweep's dominant op (largest time)
PROBE_COPY_BYTES = 256 << 20


def _copy_calibration(torch, dev):
    """A plain device copy of 256 MiB, five times: FETCH_SIZE / WRITE_SIZE of
    a known byte count, to scale the counters of the probed kernels."""
    src = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()


def kernel_probe(torch, dev, what):
    """Launches for hardware-counter passes, then the copy calibration."""
    from akas_amd import moe, ops

    info = dict(probe=what, copy_bytes=PROBE_COPY_BYTES)
    if what == "decode" or what.startswith("decode_m"):
        m = PROBE_M if what == "decode" else int(what[len("decode_m"):])
        if m not in DECODE_M:
            raise SystemExit(f"decode probe rows must be one of {DECODE_M}")
        copies = 20
        codes, scales = make_weights(torch, N_DEC, K_DEC, copies, 1234, dev)
        x = bf16_activations(torch, m, K_DEC, m, dev)
        out = torch.empty((m, N_DEC), dtype=torch.bfloat16, device=dev)
        ws = ops.linear_workspace(m, K_DEC, N_DEC, dev)
        for i in range(copies):
            ops.fp8_linear(x, codes[i], scales[i], out=out, workspace=ws)
        info.update(op=f"fp8_linear M={m} K={K_DEC} N={N_DEC} bf16, x20 on 20 weight copies",
                    op_bytes=dense_bytes(m, K_DEC, N_DEC))
    elif what == "prefill":
        k, n = PREFILL_SHAPES[0]
        codes, scales = make_weights(torch, n, k, 1, 7 + n, dev)
        x = bf16_activations(torch, 8192, k, 99, dev, outliers=0.0)
        out = torch.empty((8192, n), dtype=torch.bfloat16, device=dev)
        for _ in range(5):
            ops.fp8_linear(x, codes[0], scales[0], out=out)
        info.update(op=f"fp8_linear M=8192 K={k} N={n} bf16, x5", flops=2 * 8192 * k * n)
    elif what in ("moe_decode", "moe_prefill"):
        tokens, zipf = (256, False) if what == "moe_decode" else (16384, True)
        H, F, E = 2048, 1536, 64
        bank = {}
        for name, (n, k) in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
            c, sc = make_weights(torch, n, k, E, {"w1": 1, "w3": 3, "w2": 2}[name], dev)
            bank[name] = (torch.stack(c), torch.stack(sc))
            del c, sc
        wts = moe.ExpertWeights(*bank["w1"], *bank["w3"], *bank["w2"])
        rng = np.random.default_rng(0)
        x = torch.from_numpy(rng.normal(0, 1, (tokens, H)).astype(np.float32)).to(dev).to(torch.bfloat16)
        logits = rng.normal(0, 1, (tokens, E)).astype(np.float32)
        if zipf:
            logits += (-1.1 * np.log1p(rng.permutation(E))).astype(np.float32)[None, :]
        logits = torch.from_numpy(logits).to(dev)
        for _ in range(3):  # unpacked, as the bench line's MoE layers
            moe.routed_moe(x, logits, None, wts, top=4, packed=False, max_block_m=64,
                           product_dtype=torch.bfloat16, activation_dtype=torch.bfloat16,
                           contribution_dtype=torch.bfloat16)
        info.update(op=f"routed MoE layer T={tokens}{' zipf' if zipf else ''}, x3",
                    flops=6 * F * H * tokens * 4)
    elif what != "copy":
        raise SystemExit(f"unknown kernel probe {what!r}")
    torch.cuda.synchronize()
    _copy_calibration(torch, dev)
    print(json.dumps(info))


def library_ab(torch, dev, paths, rounds=6, launches=10):
    """The three prefill GEMM launches (M=8192, bf16 out, on prequantized
    codes) with each library in ``paths`` in turn, ``rounds`` times, all in
    one process on one GPU: builds compared on the same box and inputs.  A
    library is bound by its own entry points (``projection_partial``,
    ``quantize``), which every build of this path exports with the same
    signatures.  Prints one line per round and library, TFLOP/s per shape."""
    import ctypes

    from akas_amd import _lib, ops

    libs = []
    for path in paths:
        lib = ctypes.CDLL(path)
        for name in ("akas_quantize", "akas_projection_partial", "akas_quantize_weight_blocks",
                     "akas_status_string"):
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = _lib.SIGNATURES[name]
        libs.append(lib)
    bound = _lib._LIB
    inputs = []
    for (k, n) in PREFILL_SHAPES:
        codes, scales = make_weights(torch, n, k, 1, 7 + n, dev)
        x = bf16_activations(torch, 8192, k, 99, dev, outliers=0.0)
        q, qs = ops.quantize(x)
        inputs.append((k, n, codes[0], scales[0], q, qs,
                       torch.empty((8192, n), dtype=torch.bfloat16, device=dev)))
    try:
        for r in range(rounds):
            for path, lib in zip(paths, libs):
                _lib._LIB = lib
                row = dict(round=r, library=path)
                for (k, n, w, s, q, qs, out) in inputs:
                    ms = time_kernel_graph(torch, lambda i: ops.projection_partial(
                        q, qs, w, s, out=out, out_dtype=torch.bfloat16), launches)
                    row[f"K{k}_N{n}"] = round(2 * 8192 * k * n / (ms * 1e-3) / 1e12, 1)
                print(json.dumps(row), flush=True)
    finally:
        _lib._LIB = bound


def vendor_probe(torch, dev, rounds=4, reps=20):
    """hipBLASLt's FP8 GEMMs (``torch._scaled_mm`` with one scale per tensor,
    or one per row and column, applied once after the k-loop) beside this
    library's block-scaled GEMM launch, on the three prefill shapes and the
    same e4m3 codes, rounds interleaved in one process.  The vendor kernels
    skip the per-k-block scale fold that 1x128 / 128x128 block scales need,
    so they bound what an FP8 GEMM of these shapes reaches on this chip and
    data.  Prints one line per round, TFLOP/s per shape and kernel."""
    from akas_amd import ops

    inputs = []
    for (k, n) in PREFILL_SHAPES:
        codes, scales = make_weights(torch, n, k, 1, 7 + n, dev)
        x = bf16_activations(torch, 8192, k, 99, dev, outliers=0.0)
        q, qs = ops.quantize(x)
        inputs.append((k, n, codes[0], scales[0], q, qs,
                       torch.empty((8192, n), dtype=torch.bfloat16, device=dev)))
    one = torch.ones((), dtype=torch.float32, device=dev)
    for r in range(rounds):
        row = dict(round=r)
        for (k, n, w, s, q, qs, out) in inputs:
            flops = 2 * 8192 * k * n
            a8 = q.view(torch.float8_e4m3fn)
            b8 = w.view(torch.float8_e4m3fn).t()  # column-major [K, N]
            kernels = {
                "akas_gemm": lambda i: ops.projection_partial(q, qs, w, s, out=out, out_dtype=torch.bfloat16),
                "hipblaslt_tensorwise": lambda i: torch._scaled_mm(a8, b8, scale_a=one, scale_b=one,
                                                                   out_dtype=torch.bfloat16),
                "hipblaslt_rowwise": lambda i: torch._scaled_mm(
                    a8, b8, scale_a=torch.ones((8192, 1), dtype=torch.float32, device=dev),
                    scale_b=torch.ones((1, n), dtype=torch.float32, device=dev), out_dtype=torch.bfloat16),
            }
            for name, fn in kernels.items():
                try:
                    fn(0)
                    torch.cuda.synchronize()
                    ms = time_kernel(torch, fn, reps)
                    row[f"K{k}_N{n}_{name}"] = round(flops / (ms * 1e-3) / 1e12, 1)
                except RuntimeError as e:  # a refusal by the library, not a GPU fault
                    row[f"K{k}_N{n}_{name}"] = f"unavailable: {str(e)[:120]}"
        print(json.dumps(row), flush=True)


OPERAND_CODES = {"random": None, "zero": 0x00, "one": 0x38, "max": 0x7E}


def operand_probe(torch, dev, rounds=3, launches=10):
    """The prefill GEMM launch (M=8192, K=2048, N=6144, bf16 out) on random
    e4m3 operands and on constant ones (every code 0x00, 0x38 = 1.0 or
    0x7E = 448), interleaved over ``rounds``: identical instructions and
    addresses, different data.  Each line is TFLOP/s from HIP events around a
    graph of ``launches`` launches.  Under rocprofv3 --pmc GRBM_GUI_ACTIVE
    with --kernel-trace, the clock the chip ran at is GRBM_GUI_ACTIVE / 8 XCDs
    over each dispatch's duration."""
    from akas_amd import ops

    m, (k, n) = 8192, PREFILL_SHAPES[0]
    codes, scales = make_weights(torch, n, k, 1, 7 + n, dev)
    x = bf16_activations(torch, m, k, 99, dev, outliers=0.0)
    q, qs = ops.quantize(x)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    operands = {}
    for name, code in OPERAND_CODES.items():
        operands[name] = ((q, codes[0]) if code is None else
                          (torch.full_like(q, code), torch.full_like(codes[0], code)))
    flops = 2 * m * k * n
    for r in range(rounds):
        row = dict(round=r)
        for name, (a, w) in operands.items():
            ms = time_kernel_graph(torch, lambda i: ops.projection_partial(
                a, qs, w, scales[0], out=out, out_dtype=torch.bfloat16), launches)
            row[name] = round(flops / (ms * 1e-3) / 1e12, 1)
        print(json.dumps(row), flush=True)


def roofline_ceilings(torch, dev):
    """The GPU's measured ceilings from the probe library: a streaming read
    of 1 GiB (four times the 256 MB last-level cache) at several grid sizes,
    and back-to-back FP8 MFMAs at 8 waves per SIMD; each the best of 5 timed
    launches (HIP events on the launching stream).  Also the floor of one
    decode op: a pure read of one N x K weight matrix of the sweep in one
    launch, graph-replayed back to back over copies rotated past the
    last-level cache as the sweep's weights are (best grid)."""
    import ctypes

    from akas_amd import build

    lib = ctypes.CDLL(build.PROBE_LIBRARY)
    lib.akas_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_void_p]
    lib.akas_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.akas_probe_mfma_flops.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.akas_probe_mfma_flops.restype = ctypes.c_double
    nbytes = 1 << 30
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    best_read = (0.0, 0)
    for blocks in (1024, 2048, 4096, 8192):
        sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
        stream = torch.cuda.current_stream().cuda_stream
        ms = time_kernel(torch, lambda i: lib.akas_probe_stream_read(
            buf.data_ptr(), nbytes, sink.data_ptr(), blocks, stream), 5)
        gbs = nbytes / (ms * 1e-3) / 1e9
        best_read = max(best_read, (gbs, blocks))
    del buf
    wbytes, copies = N_DEC * K_DEC, 48
    wbufs = torch.ones((copies, wbytes // 4), dtype=torch.float32, device=dev)
    best_op = (float("inf"), 0)
    for blocks in (256, 512, 768, 1024, 2048):
        sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
        ms = time_kernel_graph(torch, lambda i: lib.akas_probe_stream_read(
            wbufs[i % copies].data_ptr(), wbytes, sink.data_ptr(), blocks,
            torch.cuda.current_stream().cuda_stream), copies)
        best_op = min(best_op, (ms * 1e3, blocks))
    del wbufs
    lib.akas_probe_load_mix.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p]
    # The split GEMM's loads alone (M = 64 and 256), over the same rotation of
    # weight copies, with row-major (as projection_partial reads them) and
    # fragment-major (as fp8_linear's quantizer writes them) activations.
    wbufs = torch.randint(0, 256, (copies, wbytes), dtype=torch.uint8, device=dev)
    load_mix = {}
    for m in (64, 256):
        acts = torch.randint(0, 256, ((m + 15) // 16 * 16 * K_DEC,), dtype=torch.uint8, device=dev)
        sink = torch.empty(2048 * 512, dtype=torch.int32, device=dev)
        row = {}
        for af, key in ((0, "row_major_us"), (1, "fragment_major_us")):
            ms = time_kernel_graph(torch, lambda i: lib.akas_probe_load_mix(
                wbufs[i % copies].data_ptr(), acts.data_ptr(), m, N_DEC, af, sink.data_ptr(), None,
                torch.cuda.current_stream().cuda_stream), copies)
            row[key] = round(ms * 1e3, 3)
        load_mix[f"M{m}"] = row
    del wbufs
    iters, blocks = 4000, 256 * 8
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    ms = time_kernel(torch, lambda i: lib.akas_probe_mfma(sink.data_ptr(), iters, blocks, stream), 5)
    tflops = lib.akas_probe_mfma_flops(iters, blocks) / (ms * 1e-3) / 1e12
    return dict(hbm_read_gbs=round(best_read[0], 1), hbm_read_grid=best_read[1],
                hbm_read_frac_of_peak=round(best_read[0] / HBM_PEAK_GBS, 4),
                mfma_fp8_tflops=round(tflops, 1),
                mfma_fp8_frac_of_peak=round(tflops / FP8_PEAK_TFLOPS, 4),
                decode_weight_read_us=round(best_op[0], 3), decode_weight_read_grid=best_op[1],
                decode_weight_read_gbs=round(wbytes / (best_op[0] * 1e-6) / 1e9, 1),
                decode_step_read_floor_us=round(len(DECODE_M) * best_op[0], 3),
                split_gemm_loads_alone=load_mix,
                source="akas_amd/csrc/probe/roofline.hip")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-probe", default=None,
                    help="only launch one workload and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--roofline-probe", action="store_true",
                    help="only measure the streaming-read and FP8 MFMA ceilings")
    ap.add_argument("--operand-probe", action="store_true",
                    help="only time the prefill GEMM on random against constant operands")
    ap.add_argument("--vendor-probe", action="store_true",
                    help="only time hipBLASLt's FP8 GEMMs beside the prefill GEMM launch")
    ap.add_argument("--library-ab", nargs="+", metavar="LIB", default=None,
                    help="only time the prefill GEMMs with each of these library builds in turn")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported "
              "(this path has no multi-GPU component)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        raise SystemExit("--steps must be >= 1 and --warmup >= 0")

    import torch

    from akas_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.kernel_probe:
        kernel_probe(torch, dev, args.kernel_probe)
        return
    if args.roofline_probe:
        print(json.dumps(roofline_ceilings(torch, dev)))
        return
    if args.operand_probe:
        operand_probe(torch, dev)
        return
    if args.library_ab:
        library_ab(torch, dev, args.library_ab)
        return
    if args.vendor_probe:
        vendor_probe(torch, dev)
        return

    dec = decode_sweep(torch, dev, args.steps, args.warmup)
    value = dec["step_bytes"] / dec["step_s"] / 1e9
    # the dominant op of the step: the largest time
    dom = max(dec["per_m"], key=lambda r: r["op_us"])
    traffic = profile_value(DECODE_COUNTERS, "traffic_bytes_per_op") if dom["M"] == PROBE_M else None
    roofline = dict(bound="hbm", achieved=dom["op_gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(dom["op_gbs"] / HBM_PEAK_GBS, 4),
                    traffic=int(traffic) if traffic else None,
                    kernel=f"fp8_linear op at M={dom['M']}, K={K_DEC}, N={N_DEC}, bf16 in and out "
                           f"(every launch it makes, as the step runs it)",
                    bytes_per_launch=dom["op_bytes"], avg_us=dom["op_us"],
                    traffic_source=f"profiles/{DECODE_COUNTERS}" if traffic else None)
    line = dict(metric=METRIC, value=round(value, 1), unit="GB/s", n_gpus=1, steps=dec["steps"],
                warmup=args.warmup, ms_per_step=round(dec["step_s"] * 1e3, 4),
                higher_is_better=True, scaling="weak", vs_baseline=None, dtype="fp8e4m3xfp8e4m3->f32",
                data="synthetic",
                config=dict(workload="decode-shape dense FP8 linear sweep", M=list(DECODE_M),
                            K=K_DEC, N=N_DEC, x="bf16 ~N(0,1), 1% x20", w="e4m3 N(0,0.02), "
                            "128x128 f32 block scales", out="bf16",
                            weight_copies_rotated=dec["copies"],
                            weight_copies_read_in_timed_region=dec["touched"],
                            weight_copy_bytes=N_DEC * K_DEC),
                roofline=roofline, sweep=dec["per_m"])
    line["ceilings"] = roofline_ceilings(torch, dev)
    if not args.no_extras:
        prefill = prefill_gemms(torch, dev, 20)
        top = prefill[0]
        busy = profile_value(PREFILL_COUNTERS, "mfma_busy_frac")
        traffic = profile_value(PREFILL_COUNTERS, "traffic_bytes_per_op")
        line["roofline_prefill"] = dict(
            bound="mfma", achieved=top["op_tflops"], peak=FP8_PEAK_TFLOPS, unit="TFLOP/s",
            frac=round(top["op_tflops"] / FP8_PEAK_TFLOPS, 4),
            traffic=int(traffic) if traffic else None,
            kernel=f"fp8_linear op at M=8192, K={top['K']}, N={top['N']}, bf16 in and out (its "
                   f"quantizer launch and its GEMM launch)",
            flops_per_launch=2 * 8192 * top["K"] * top["N"], avg_us=top["op_us"],
            gemm_launch_us=top["gemm_us"], gemm_launch_frac=top["gemm_frac_fp8"],
            mfma_busy_frac=busy,
            counters_source=f"profiles/{PREFILL_COUNTERS}" if busy or traffic else None)
        line["extras"] = dict(
            config1_linear=config1_linear_bench(torch, dev),
            prefill_gemm=prefill,
            moe_decode=moe_layer_bench(torch, dev, 256, False, 20),
            moe_decode_packed=moe_layer_bench(torch, dev, 256, False, 20, packed=True),
            moe_prefill_zipf=moe_layer_bench(torch, dev, 16384, True, 10),
            moe_prefill_zipf_packed=moe_layer_bench(torch, dev, 16384, True, 10, packed=True),
            rms_quantize=rms_quantize_bench(torch, dev),
            shared_expert_moe_decode=shared_expert_block_bench(torch, dev))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
