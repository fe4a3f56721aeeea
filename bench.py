"""Benchmark of the block-scaled FP8 path on one MI355X.

Headline workload: the decode-shape dense FP8 linear sweep -- bf16
activations ``[M, 2048]`` (~N(0,1), 1% of entries x20) for M in
{1, 4, 16, 64, 256} against e4m3 weights ``[6144, 2048]`` with 128x128 f32
block scales; one step = one ``fp8_linear`` (1x128 quantize + block-scaled
MFMA GEMM, bf16 out) per M.  The value is whole-step algorithmic HBM bytes
per second, ``sum_M N*K + 4*ceil(N/128)*K/128 + 2*M*K + 2*M*N`` over the
step time.  Every step reads a different copy of the weights (more than
512 MB of copies in rotation), so weights stream from HBM, not from the
256 MB last-level cache.

Also reported (``extras``): the prefill-shape GEMMs (M=8192), the MoE decode
layer (T=256), the skewed MoE prefill layer (T=16384), the fused RMSNorm +
quantizer (16384 x 2048) and the shared-expert (Qwen3.5 block-fp8) MoE block
at decode (T=64, 256 experts, top 8), in TFLOP/s and GB/s, each block timed
as one of four captured back to back in a graph (as a decode step graph holds
many layers); ``roofline`` for the dominant kernel (HIP-event timing of that kernel
alone); ``cpu_baseline`` from the oracle's C restatement on the host cores.

    python bench.py [--steps K] [--warmup W] [--no-extras] [--no-cpu]
    python bench.py --kernel-probe    # launches for rocprofv3 --pmc passes
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


def decode_sweep(torch, dev, steps, warmup):
    from akas_amd import ops

    wbytes = N_DEC * K_DEC
    copies = max(8, math.ceil(640e6 / wbytes))
    codes, scales = make_weights(torch, N_DEC, K_DEC, copies, 1234, dev)
    xs = {m: bf16_activations(torch, m, K_DEC, m, dev) for m in DECODE_M}
    outs = {m: torch.empty((m, N_DEC), dtype=torch.bfloat16, device=dev) for m in DECODE_M}
    ws = ops.linear_workspace(max(DECODE_M), K_DEC, N_DEC, dev)
    step_bytes = sum(dense_bytes(m, K_DEC, N_DEC) for m in DECODE_M)

    def step(i):
        c, s = codes[i % copies], scales[i % copies]
        for m in DECODE_M:
            ops.fp8_linear(xs[m], c, s, out=outs[m], workspace=ws)

    # one graph replay = `copies` steps, each on a different weight copy
    g = graph_of(torch, step, copies)
    replays = max(1, math.ceil(steps / copies))
    for _ in range(max(1, math.ceil(warmup / copies))):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        g.replay()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / (replays * copies)

    # per-M GEMM kernel durations (prequantized path = the same GEMM kernel)
    per_m = []
    for m in DECODE_M:
        q, qs = ops.quantize(xs[m])
        ms = time_kernel_graph(torch, lambda i: ops.projection_partial(
            q, qs, codes[i % copies], scales[i % copies], out=outs[m],
            out_dtype=torch.bfloat16), copies)
        b = gemm_kernel_bytes(m, K_DEC, N_DEC)
        per_m.append(dict(M=m, kernel_us=round(ms * 1e3, 3), bytes=b,
                          gbs=round(b / (ms * 1e-3) / 1e9, 1),
                          frac_hbm=round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                          tflops=round(2 * m * K_DEC * N_DEC / (ms * 1e-3) / 1e12, 2)))
    return dict(step_s=dt, step_bytes=step_bytes, per_m=per_m, copies=copies,
                steps=replays * copies)


def prefill_gemms(torch, dev, steps):
    from akas_amd import ops

    res = []
    for (k, n) in ((2048, 6144), (2048, 8192), (8192, 2048)):
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
        res.append(dict(M=m, K=k, N=n, op_us=round(ms_total * 1e3, 2),
                        gemm_us=round(ms_gemm * 1e3, 2),
                        op_tflops=round(flops / (ms_total * 1e-3) / 1e12, 1),
                        gemm_tflops=round(flops / (ms_gemm * 1e-3) / 1e12, 1),
                        gemm_frac_fp8=round(flops / (ms_gemm * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4)))
        del codes, scales, x, out
    return res


LAYERS_PER_GRAPH = 4  # MoE blocks captured back to back in one graph


def moe_layer_bench(torch, dev, tokens, zipf, steps):
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
    packed = tokens >= 2048
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
    return dict(T=tokens, zipf=zipf, us=round(ms * 1e3, 2),
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


def cpu_baseline(budget_s=12.0):
    """The oracle's C restatement of the decode sweep on the host cores."""
    import ctypes

    from oracle import native
    from oracle import fp8 as ofp8

    lib = native.load()
    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "16")), 16)
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (N_DEC, K_DEC)).astype(np.float32)
    codes, scales = ofp8.quantize_weight_blocks(w)
    xs = {m: ofp8.bf16_bits(rng.normal(0, 1, (m, K_DEC)).astype(np.float32)) for m in DECODE_M}
    outs = {m: np.empty((m, N_DEC), np.uint16) for m in DECODE_M}

    def sweep():
        for m in DECODE_M:
            lib.ref_fp8_linear_bf16(native.ptr(xs[m]), native.ptr(codes), native.ptr(scales),
                                    native.ptr(outs[m]), 1, m, K_DEC, N_DEC, threads)

    sweep()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        sweep()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    step_bytes = sum(dense_bytes(m, K_DEC, N_DEC) for m in DECODE_M)

    # One thread as well (the reference's CI runs its CPU checks with
    # OMP_NUM_THREADS=1): median of 5 sweeps.
    def sweep1():
        for m in DECODE_M:
            lib.ref_fp8_linear_bf16(native.ptr(xs[m]), native.ptr(codes), native.ptr(scales),
                                    native.ptr(outs[m]), 1, m, K_DEC, N_DEC, 1)

    times1 = []
    for _ in range(5):
        t0 = time.perf_counter()
        sweep1()
        times1.append(time.perf_counter() - t0)
    med1 = float(np.median(times1))
    return dict(value=round(step_bytes / med / 1e9, 2), unit="GB/s", cores=threads,
                kind="port", cpu_model=_cpu_model(), host_cpus=os.cpu_count(),
                sample=f"full decode sweep (M=1,4,16,64,256; K=2048; N=6144), median of "
                       f"{len(times)} runs, {med * 1e3:.1f} ms/sweep, oracle/cpu_ref.c -O3 "
                       f"-fopenmp f32 accumulation",
                value_1_thread=round(step_bytes / med1 / 1e9, 3),
                sample_1_thread=f"same sweep on 1 thread, median of 5 runs, "
                                f"{med1 * 1e3:.1f} ms/sweep")


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_gemm_m256_counters.md")


def measured_traffic():
    """HBM bytes per launch of the dominant decode GEMM from the committed
    FETCH_SIZE / WRITE_SIZE summary (calibrated against a copy of known
    size), or None when the summary is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


PROBE_M = 256          # the sweep's dominant GEMM (largest kernel time)
PROBE_COPY_BYTES = 256 << 20


def kernel_probe(torch, dev):
    """Launches for hardware-counter runs: the dominant decode GEMM (M=256,
    prequantized input, bf16 out, each launch on a different weight copy) 20
    times, then a plain 256 MiB device copy 5 times, whose FETCH_SIZE /
    WRITE_SIZE calibrate the counters against a known byte count."""
    from akas_amd import ops

    copies = 20
    codes, scales = make_weights(torch, N_DEC, K_DEC, copies, 1234, dev)
    x = bf16_activations(torch, PROBE_M, K_DEC, PROBE_M, dev)
    q, qs = ops.quantize(x)
    out = torch.empty((PROBE_M, N_DEC), dtype=torch.bfloat16, device=dev)
    for i in range(copies):
        ops.projection_partial(q, qs, codes[i], scales[i], out=out, out_dtype=torch.bfloat16)
    src = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps(dict(probe="decode GEMM M=256 K=2048 N=6144 x20, then 256 MiB copy x5",
                          gemm_bytes_per_launch=gemm_kernel_bytes(PROBE_M, K_DEC, N_DEC),
                          copy_bytes=PROBE_COPY_BYTES)))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-probe", action="store_true",
                    help="only launch the dominant kernel and a calibration copy (for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported "
              "(this path has no multi-GPU component)", file=sys.stderr)
        sys.exit(2)

    import torch

    from akas_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.kernel_probe:
        kernel_probe(torch, dev)
        return

    dec = decode_sweep(torch, dev, args.steps, args.warmup)
    value = dec["step_bytes"] / dec["step_s"] / 1e9
    # dominant kernel: the largest share of the sweep's GEMM time
    dom = max(dec["per_m"], key=lambda r: r["kernel_us"])
    traffic = measured_traffic() if dom["M"] == PROBE_M else None
    roofline = dict(bound="hbm", achieved=dom["gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(dom["gbs"] / HBM_PEAK_GBS, 4), traffic=traffic,
                    kernel=f"GEMM launch at M={dom['M']}, K={K_DEC}, N={N_DEC}",
                    bytes_per_launch=dom["bytes"], avg_us=dom["kernel_us"],
                    traffic_source=os.path.relpath(TRAFFIC_PROFILE, ROOT) if traffic else None)
    line = dict(metric=METRIC, value=round(value, 1), unit="GB/s", n_gpus=1, steps=dec["steps"],
                warmup=args.warmup, ms_per_step=round(dec["step_s"] * 1e3, 4),
                higher_is_better=True, scaling="weak", vs_baseline=None, dtype="fp8e4m3xfp8e4m3->f32",
                data="synthetic",
                config=dict(workload="decode-shape dense FP8 linear sweep", M=list(DECODE_M),
                            K=K_DEC, N=N_DEC, x="bf16 ~N(0,1), 1% x20", w="e4m3 N(0,0.02), "
                            "128x128 f32 block scales", out="bf16",
                            weight_copies_rotated=dec["copies"]),
                roofline=roofline, sweep=dec["per_m"])
    if not args.no_extras:
        line["extras"] = dict(
            prefill_gemm=prefill_gemms(torch, dev, 20),
            moe_decode=moe_layer_bench(torch, dev, 256, False, 20),
            moe_prefill_zipf=moe_layer_bench(torch, dev, 16384, True, 10),
            rms_quantize=rms_quantize_bench(torch, dev),
            shared_expert_moe_decode=shared_expert_block_bench(torch, dev))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
