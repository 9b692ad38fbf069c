#!/usr/bin/env python3
"""Benchmark of the gfx950 packed-weight matmul path on one MI355X.

Headline: Q4_K decode GEMV x[1, 4096] . W[14336, 4096]^T (Llama-3-8B FFN up
projection), weight GB/s over quantized-weight bytes. A step is one call
of the matmul entry point (int8 activation quantization + GEMV) on inputs
already resident in HBM; the weight rotates through `--copies` distinct
device copies (> 256 MB in all) so the MALL cannot serve it. Steps are
launched from HIP graphs (captured once) so host launch cost does not hide
the device time.

Also reported: the GEMV kernel alone against the 8 TB/s HBM roofline and
against a streaming-read ceiling measured in the same run (`extra`), the
GEMV at m = 2, 4, 8 and the IQ4_XS down projection, one Llama-3-8B-shaped
decoder layer decode step (device-resident, weights + KV cache bytes per
step, rotated over several layer copies), the same GEMV and GEMM for the
other formats, the M=512 prefill GEMM (x[512, 4096] . W[14336, 4096]^T) in
TFLOP/s against the 2.5 PFLOP/s dense f16 MFMA peak with the prefill
shapes around it, and the reference's CPU path (the oracle's restatement
of its column kernels) timed on this host's cores: the headline workload
and legs for the 4096 x 4096 matvec, the M=512 GEMM and the IQ4_XS GEMV
(`cpu_baseline.legs`).
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "magnetar-provider-cpu_amd"))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV weight GB/s (% HBM peak) + M=512 GEMM TFLOP/s, 4096x14336"
HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    """The host CPU as /proc/cpuinfo names it, with its family / model /
    stepping numbers (a virtualised host may print only the vendor line)."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                key, val = (t.strip() for t in line.split(":", 1))
                fields.setdefault(key, val)
            elif fields:
                break  # the first processor's block is enough
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    ident = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return f"{name} ({ident})" if ident else name


def affinity_threads():
    """T: the logical CPUs this process may run on (the reference sizes its
    pool by available_parallelism, which reads the same mask)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def graph_size(steps, cap):
    """Calls per captured graph: the largest divisor of `steps` not above
    `cap`, so that exactly `steps` calls are timed."""
    for d in range(max(1, min(cap, steps)), 0, -1):
        if steps % d == 0:
            return d
    return 1


class GraphRunner:
    """Captures `per_graph` calls of fn(i) into one HIP graph on a private
    stream, then replays it; falls back to eager launches if capture fails."""

    def __init__(self, torch, fn, per_graph, use_graph=True):
        self.torch = torch
        self.fn = fn
        self.per_graph = per_graph
        self.stream = torch.cuda.Stream()
        self.graph = None
        torch.cuda.synchronize()
        with torch.cuda.stream(self.stream):
            for i in range(per_graph):
                fn(i, self.stream.cuda_stream)
        self.stream.synchronize()
        if use_graph:
            try:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.stream):
                    for i in range(per_graph):
                        fn(i, self.stream.cuda_stream)
                self.graph = g
            except Exception as e:  # noqa: BLE001
                log(f"graph capture failed ({e}); timing eager launches")
                self.graph = None
        torch.cuda.synchronize()

    def run(self, calls):
        """Enqueues `calls` calls on the current stream: whole graph replays,
        then the remainder (calls % per_graph) as eager launches."""
        torch = self.torch
        cur = torch.cuda.current_stream()
        if self.graph is not None:
            for _ in range(calls // self.per_graph):
                self.graph.replay()
            for i in range(calls % self.per_graph):
                self.fn(i, cur.cuda_stream)
        else:
            for i in range(calls):
                self.fn(i, cur.cuda_stream)

    def time(self, calls):
        """Seconds for `calls` calls, HIP events on the launching stream."""
        torch = self.torch
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        self.run(calls)
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / 1e3


def round_up(v, m):
    return (v + m - 1) // m * m


def warm(runner, per, seconds=0.05):
    """Untimed replays of `per` calls until `seconds` of GPU time have run.
    The prefill GEMMs need tens of milliseconds of load before their time
    settles: after a 10-call warm-up 512 x 14336 x 4096 read 76.5 us, after
    one more 60-call round 66.7 us."""
    spent = 0.0
    while spent < seconds:
        spent += runner.time(per)


def recorded_traffic(name):
    """HBM bytes per launch of kernel `name` as measured by the two
    rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE, calibrated against a
    plain copy) summarised under profiles/, or None if not recorded."""
    import glob
    import re

    pat = re.compile(rf"^traffic_bytes_per_launch {re.escape(name)} = (\d+)\s*$")
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        for line in open(path):
            m = pat.match(line)
            if m:
                return int(m.group(1))
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=10, help="distinct weight copies rotated through")
    ap.add_argument("--per-graph", type=int, default=100, help="calls captured per HIP graph")
    ap.add_argument("--gemm-steps", type=int, default=50)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="bound on CPU-baseline timing")
    ap.add_argument("--parts", default="gemv,stream,shapes,iq4xs,layer,formats,gemm,cpu",
                    help="comma list of parts to run (the headline line needs gemv)")
    ap.add_argument("--layer-copies", type=int, default=3,
                    help="decoder-layer copies the decode step rotates through (> 256 MB in all)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="also run a plain device copy of this size (counter calibration under rocprofv3)")
    args = ap.parse_args()
    parts = set(args.parts.split(","))
    if args.no_cpu:
        parts.discard("cpu")

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path runs on a single MI355X and takes no "
              f"multi-GPU figure (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import magnetar_gpu as mg
    from magnetar_gpu import workloads

    torch.cuda.set_device(0)
    ctx = mg.Context(0)
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be at least 1 and --warmup at least 0", file=sys.stderr)
        sys.exit(2)
    # exactly --steps timed calls and --warmup untimed ones for the headline
    steps, warmup = args.steps, args.warmup
    per_graph = graph_size(steps, args.per_graph)

    # ---- decode GEMV: Q4_K x[1, 4096] . W[14336, 4096]^T -------------------------
    name = "q4k_14336x4096_s1"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    wbytes = workloads.weight_bytes(name)
    weight_bytes = workloads.weight_bytes_per_call(name)
    copies = [ctx.upload(fmt, n, k, wbytes) for _ in range(args.copies)]
    x_host = workloads.activations(seed, 1, k)
    x = torch.from_numpy(x_host).cuda()
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    xq = torch.empty(k, dtype=torch.int8, device="cuda")
    xs = torch.empty(k // 32, dtype=torch.float32, device="cuda")
    xh = torch.empty(k // 16, dtype=torch.int32, device="cuda")
    log(f"gemv: {name}, {weight_bytes} weight bytes x {args.copies} copies "
        f"({args.copies * weight_bytes / 2**20:.0f} MiB rotated)")

    def step(i, stream):
        ctx.matmul_dev(copies[i % len(copies)], x.data_ptr(), 1, k, y.data_ptr(), int8=True, stream=stream)

    def gemv_only(i, stream):
        ctx.matmul_prequantized_dev(copies[i % len(copies)], xq.data_ptr(), xs.data_ptr(), xh.data_ptr(), 1, k,
                                    y.data_ptr(), stream=stream)

    ctx.quantize_activations_dev(x.data_ptr(), 1, k, xq.data_ptr(), xs.data_ptr(), xh.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream)
    use_graph = not args.no_graph
    step_runner = GraphRunner(torch, step, per_graph, use_graph)
    step_runner.run(warmup)
    t_step = step_runner.time(steps)
    ms_per_step = t_step / steps * 1e3
    value = weight_bytes * steps / t_step / 1e9
    log(f"gemv step (quantize + GEMV): {ms_per_step * 1e3:.2f} us/step, {value:.1f} GB/s")

    # The step is one launch (int8 quantization fused into the GEMV for
    # m <= 4), so the roofline's kernel time is the step's launch time.
    kernel_us = t_step / steps * 1e6
    achieved = weight_bytes / (kernel_us * 1e-6) / 1e9
    log(f"gemv kernel (fused quantize + GEMV): {kernel_us:.2f} us, {achieved:.1f} GB/s = "
        f"{achieved / HBM_PEAK_GBS:.3f} of HBM peak")
    kernel_runner = GraphRunner(torch, gemv_only, per_graph, use_graph)
    kernel_runner.run(max(warmup, per_graph))
    t_pre = kernel_runner.time(steps) / steps
    log(f"gemv on pre-quantized activations: {t_pre * 1e6:.2f} us, {weight_bytes / t_pre / 1e9:.1f} GB/s")

    # parity spot check of the timed path against the oracle
    torch.cuda.synchronize()
    step(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    y_gpu = y.cpu().numpy()

    if args.copy_calibration_mib:
        nbytes = args.copy_calibration_mib << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: 5 plain copies of {nbytes} bytes (read {nbytes}, write {nbytes} per copy)")

    # ---- other decode shapes (kernel alone) --------------------------------------
    extra = {"q4k_gemv_prequantized_kernel_us": round(t_pre * 1e6, 3),
             "q4k_gemv_prequantized_GBps": round(weight_bytes / t_pre / 1e9, 1)}
    for m in ((2, 4, 8) if "shapes" in parts else ()):
        xm = torch.from_numpy(workloads.activations(seed, m, k)).cuda()
        qv = torch.empty(m * k, dtype=torch.int8, device="cuda")
        qs = torch.empty(m * k // 32, dtype=torch.float32, device="cuda")
        qh = torch.empty(m * k // 16, dtype=torch.int32, device="cuda")
        ym = torch.empty((m, n), dtype=torch.float32, device="cuda")
        ctx.quantize_activations_dev(xm.data_ptr(), m, k, qv.data_ptr(), qs.data_ptr(), qh.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream)

        def gm(i, stream, m=m, qv=qv, qs=qs, qh=qh, ym=ym):
            ctx.matmul_prequantized_dev(copies[i % len(copies)], qv.data_ptr(), qs.data_ptr(), qh.data_ptr(), m,
                                        k, ym.data_ptr(), stream=stream)

        r = GraphRunner(torch, gm, per_graph, use_graph)
        r.time(per_graph)
        t = r.time(5 * per_graph) / (5 * per_graph)
        extra[f"q4k_gemv_m{m}_kernel_us"] = round(t * 1e6, 3)
        extra[f"q4k_gemv_m{m}_GBps"] = round(weight_bytes / t / 1e9, 1)
        log(f"gemv m={m} kernel: {t * 1e6:.2f} us, {weight_bytes / t / 1e9:.1f} GB/s")

    if "stream" in parts:
        stream_part(torch, weight_bytes, args.copies, kernel_us, extra)
    if "iq4xs" in parts:
        iq4xs_part(ctx, torch, workloads, args, per_graph, use_graph, extra)
    if "layer" in parts:
        layer_part(ctx, torch, per_graph, use_graph, extra, args.layer_copies)
    if "formats" in parts:
        formats_part(ctx, torch, per_graph, use_graph, extra)
    gemm = gemm_part(ctx, torch, workloads, use_graph, args) if "gemm" in parts else None
    cpu = cpu_part(fmt, wbytes, n, k, x_host, y_gpu, weight_bytes, args, kernel_us, gemm, extra) \
        if "cpu" in parts else None

    for h in copies:
        h.release()
    ctx.close()
    emit(args, value, steps, warmup, ms_per_step, n, k, weight_bytes, use_graph, step_runner, achieved, kernel_us,
         cpu, gemm, extra)


def stream_part(torch, nbytes, copies, gemv_us, extra):
    """The practical read ceiling at the GEMV's size: a kernel that only
    reads `nbytes` (the headline weight's bytes) with 16-byte loads, rotated
    over as many distinct buffers as the GEMV's weight copies (so the MALL
    cannot serve it), best over a small sweep of launch shapes."""
    import magnetar_gpu as mg

    L = mg.probe_lib()
    bufs = [torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device="cuda") for _ in range(copies)]
    best = None
    for loads in (1, 2, 4, 8):
        for block in (256, 512):
            sink = torch.zeros(int(L.mqp_stream_groups(nbytes, loads, block)), dtype=torch.int32, device="cuda")

            def read(i, stream, loads=loads, block=block, sink=sink):
                rc = L.mqp_stream_read(bufs[i % len(bufs)].data_ptr(), nbytes, loads, block, sink.data_ptr(), stream)
                if rc:
                    raise RuntimeError("stream-read probe launch failed")

            r = GraphRunner(torch, read, 100, True)
            r.run(100)
            t = r.time(500) / 500
            if best is None or t < best[0]:
                best = (t, loads, block)
    t, loads, block = best
    extra["stream_read_ceiling_us"] = round(t * 1e6, 3)
    extra["stream_read_ceiling_GBps"] = round(nbytes / t / 1e9, 1)
    extra["stream_read_ceiling_frac_hbm"] = round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)
    extra["stream_read_ceiling_shape"] = f"{nbytes} B x {copies} buffers, {loads} x 16 B per lane, {block} threads"
    extra["gemv_frac_of_stream_ceiling"] = round(t * 1e6 / gemv_us, 4)
    log(f"streaming-read ceiling at {nbytes} B: {t * 1e6:.2f} us, {nbytes / t / 1e9:.1f} GB/s "
        f"({loads} loads/lane, {block} threads); the GEMV step reaches {t * 1e6 / gemv_us:.3f} of it")
    del bufs


def iq4xs_part(ctx, torch, workloads, args, per_graph, use_graph, extra):
    # IQ4_XS GEMV x[1, 14336] . W[4096, 14336]^T
    iname = "iq4xs_4096x14336_s3"
    ifmt, inn, ik, iseed, _ = workloads.WEIGHTS[iname]
    ibytes = workloads.weight_bytes_per_call(iname)
    iw = workloads.weight_bytes(iname)
    icopies = [ctx.upload(ifmt, inn, ik, iw) for _ in range(args.copies)]
    ix = torch.from_numpy(workloads.activations(iseed, 1, ik)).cuda()
    iq = torch.empty(ik, dtype=torch.int8, device="cuda")
    isc = torch.empty(ik // 32, dtype=torch.float32, device="cuda")
    ish = torch.empty(ik // 16, dtype=torch.int32, device="cuda")
    iy = torch.empty((1, inn), dtype=torch.float32, device="cuda")
    ctx.quantize_activations_dev(ix.data_ptr(), 1, ik, iq.data_ptr(), isc.data_ptr(), ish.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream)

    def ig(i, stream):
        ctx.matmul_prequantized_dev(icopies[i % len(icopies)], iq.data_ptr(), isc.data_ptr(), ish.data_ptr(), 1, ik,
                                    iy.data_ptr(), stream=stream)

    r = GraphRunner(torch, ig, per_graph, use_graph)
    r.time(per_graph)
    t = r.time(5 * per_graph) / (5 * per_graph)
    extra["iq4xs_gemv_kernel_us"] = round(t * 1e6, 3)
    extra["iq4xs_gemv_GBps"] = round(ibytes / t / 1e9, 1)
    extra["iq4xs_gemv_frac_hbm"] = round(ibytes / t / 1e9 / HBM_PEAK_GBS, 4)
    log(f"iq4xs gemv kernel: {t * 1e6:.2f} us, {ibytes / t / 1e9:.1f} GB/s")
    for h in icopies:
        h.release()


def layer_part(ctx, torch, per_graph, use_graph, extra, copies):
    # ---- one Llama-3-8B-shaped decoder layer decode step (seed 4) ----------------
    # fused: 6 launches (mq_decode_matmul_dev); unfused: each operator's own
    # entry point, 12 launches. The step rotates through `copies` uploads of
    # the layer (weights and KV cache: 156 MB each), so successive steps
    # read distinct bytes and the 256 MB MALL cannot hold the working set.
    from magnetar_gpu import decoder

    data = decoder.LayerData(seed=4)
    position = data.prefilled  # the token after the 4095 cached ones
    kv_bytes = 2 * (position + 1) * decoder.KV_HEADS * decoder.HEAD_DIM * 4
    hbm = data.weight_bytes() + kv_bytes
    copies = max(2, copies)
    for fused, key in ((True, "layer_decode_step"), (False, "layer_decode_step_unfused")):
        layers = [decoder.DecoderLayer(ctx, torch, data, fused=fused) for _ in range(copies)]

        def step(i, stream, layers=layers):
            layers[i % len(layers)].step(position, stream=stream)

        per = 10 * copies
        r = GraphRunner(torch, step, per, use_graph)
        r.time(per)
        calls = 10 * per
        t = r.time(calls) / calls
        extra[f"{key}_us"] = round(t * 1e6, 2)
        extra[f"{key}_GBps"] = round(hbm / t / 1e9, 1)
        extra[f"{key}_frac_hbm"] = round(hbm / t / 1e9 / HBM_PEAK_GBS, 4)
        log(f"decoder layer decode step ({'fused, 6' if fused else 'unfused, 12'} launches): {t * 1e6:.1f} us, "
            f"{hbm} HBM bytes (Q4_K weights {data.weight_bytes()} + f32 K/V {kv_bytes}), {hbm / t / 1e9:.1f} GB/s, "
            f"rotated over {copies} layer copies ({copies * hbm / 2**20:.0f} MiB)")
        for layer in layers:
            layer.release()
        del layers
        torch.cuda.empty_cache()
    extra["layer_decode_step_bytes"] = hbm
    extra["layer_decode_step_copies"] = copies


def formats_part(ctx, torch, per_graph, use_graph, extra):
    # ---- the plane formats: decode GEMV x[1, 4096] . W[14336, 4096]^T and the
    # M = 512 prefill GEMM on the same weight (random blocks, small f16 scales)
    import magnetar_gpu as mg
    from magnetar_gpu import workloads

    n, k = 14336, 4096
    x = torch.from_numpy(mg.gaussian(4500, 1.0, k).reshape(1, k)).cuda()
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    xm = torch.from_numpy(mg.gaussian(4501, 1.0, 512 * k).reshape(512, k)).cuda()
    ym = torch.empty((512, n), dtype=torch.float32, device="cuda")
    for fmt in (mg.Q8_0, mg.Q6_K, mg.Q5_K, mg.Q4_0, mg.IQ4_NL, mg.Q3_K, mg.Q2_K):
        name = mg.FORMAT_NAMES[fmt]
        w = workloads.random_blocks(fmt, n, k, 4000 + fmt)
        copies = [ctx.upload(fmt, n, k, w) for _ in range(max(2, -(-600_000_000 // w.size)))]

        def gv(i, stream, copies=copies):
            ctx.matmul_dev(copies[i % len(copies)], x.data_ptr(), 1, k, y.data_ptr(), int8=True, stream=stream)

        r = GraphRunner(torch, gv, per_graph, use_graph)
        r.time(per_graph)
        t = r.time(5 * per_graph) / (5 * per_graph)
        extra[f"{name}_gemv_kernel_us"] = round(t * 1e6, 3)
        extra[f"{name}_gemv_GBps"] = round(w.size / t / 1e9, 1)
        extra[f"{name}_gemv_frac_hbm"] = round(w.size / t / 1e9 / HBM_PEAK_GBS, 4)

        def gm(i, stream, copies=copies):
            ctx.matmul_dev(copies[i % len(copies)], xm.data_ptr(), 512, k, ym.data_ptr(), int8=True, stream=stream)

        rg = GraphRunner(torch, gm, 5, use_graph)
        warm(rg, 5)
        tg = rg.time(20) / 20
        tflops = 2 * 512 * n * k / tg / 1e12
        extra[f"{name}_gemm512_us"] = round(tg * 1e6, 2)
        extra[f"{name}_gemm512_TFLOPs"] = round(tflops, 1)
        log(f"{name}: gemv {t * 1e6:.2f} us, {w.size / t / 1e9:.1f} GB/s ({w.size} B); "
            f"M=512 gemm {tg * 1e6:.1f} us, {tflops:.1f} TFLOP/s")
        for h in copies:
            h.release()
    # the IQ2 / IQ3 grid formats (stand-in grid tables of the real shapes): the
    # decode GEMV and the M = 512 prefill GEMM (raw blocks decoded per lane)
    ctx.set_iq_grids(workloads.synthetic_iq_grids(1))
    for fmt in mg.GRID_FORMATS:
        name = mg.FORMAT_NAMES[fmt]
        w = workloads.random_blocks(fmt, n, k, 4000 + fmt)
        copies = [ctx.upload(fmt, n, k, w) for _ in range(max(2, -(-600_000_000 // w.size)))]

        def gv(i, stream, copies=copies):
            ctx.matmul_dev(copies[i % len(copies)], x.data_ptr(), 1, k, y.data_ptr(), int8=True, stream=stream)

        r = GraphRunner(torch, gv, per_graph, use_graph)
        r.time(per_graph)
        t = r.time(5 * per_graph) / (5 * per_graph)
        extra[f"{name}_gemv_kernel_us"] = round(t * 1e6, 3)
        extra[f"{name}_gemv_GBps"] = round(w.size / t / 1e9, 1)
        extra[f"{name}_gemv_frac_hbm"] = round(w.size / t / 1e9 / HBM_PEAK_GBS, 4)

        def gm(i, stream, copies=copies):
            ctx.matmul_dev(copies[i % len(copies)], xm.data_ptr(), 512, k, ym.data_ptr(), int8=True, stream=stream)

        rg = GraphRunner(torch, gm, 5, use_graph)
        warm(rg, 5)
        tg = rg.time(20) / 20
        tflops = 2 * 512 * n * k / tg / 1e12
        extra[f"{name}_gemm512_us"] = round(tg * 1e6, 2)
        extra[f"{name}_gemm512_TFLOPs"] = round(tflops, 1)
        log(f"{name}: gemv {t * 1e6:.2f} us, {w.size / t / 1e9:.1f} GB/s ({w.size} B); "
            f"M=512 gemm {tg * 1e6:.1f} us, {tflops:.1f} TFLOP/s")
        for h in copies:
            h.release()


def gemm_part(ctx, torch, workloads, use_graph, args):
    # ---- prefill GEMM: x[512, 4096] . W[14336, 4096]^T ---------------------------
    gname = "q4k_14336x4096_s2"
    gfmt, gn, gk, gseed, _ = workloads.WEIGHTS[gname]
    gm_rows = 512
    gw = ctx.upload(gfmt, gn, gk, workloads.weight_bytes(gname))
    gx = torch.from_numpy(workloads.activations(gseed, gm_rows, gk)).cuda()
    ga = torch.empty(gm_rows * gk + 2 * gm_rows, dtype=torch.float16, device="cuda")  # values, then row factors
    gy = torch.empty((gm_rows, gn), dtype=torch.float32, device="cuda")
    flops = 2.0 * gm_rows * gn * gk

    def gstep(i, stream):
        ctx.matmul_dev(gw, gx.data_ptr(), gm_rows, gk, gy.data_ptr(), int8=True, stream=stream)

    def gkern(i, stream):
        ctx.matmul_f16_dev(gw, ga.data_ptr(), gm_rows, gk, gy.data_ptr(), stream=stream)

    ctx.prepare_activations_f16_dev(gx.data_ptr(), gm_rows, gk, ga.data_ptr(), int8=True,
                                    stream=torch.cuda.current_stream().cuda_stream)
    gper = 10
    gsteps = round_up(max(args.gemm_steps, gper), gper)
    r = GraphRunner(torch, gstep, gper, use_graph)
    warm(r, gper)
    t_gstep = r.time(gsteps) / gsteps
    r = GraphRunner(torch, gkern, gper, use_graph)
    warm(r, gper)
    t_gkern = r.time(gsteps) / gsteps
    gemm = {
        "workload": "Q4_K prefill GEMM x[512,4096] . W[14336,4096]^T, seed 2",
        "dtype": "f16 MFMA operands (f16(q*d) int8-rounded activations, f16(s*q-m) weights), f32 accumulate",
        "step_tflops": round(flops / t_gstep / 1e12, 2),
        "ms_per_step": round(t_gstep * 1e3, 4),
        "roofline": {"bound": "mfma", "achieved": round(flops / t_gkern / 1e12, 2), "peak": F16_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / t_gkern / 1e12 / F16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": recorded_traffic("gemm_q4k_512x14336x4096"), "kernel_us": round(t_gkern * 1e6, 2),
                     "peak_basis": "dense f16 MFMA (f16 activations x f16-dequantized weights, f32 accumulate)"},
    }
    log(f"gemm m=512: step {t_gstep * 1e6:.1f} us ({flops / t_gstep / 1e12:.1f} TFLOP/s), "
        f"kernel {t_gkern * 1e6:.1f} us ({flops / t_gkern / 1e12:.1f} TFLOP/s)")
    # the prefill shapes around it (kernel time on prepared f16 activations):
    # M in {128, 512, 2048} over W[4096, 4096] and W[14336, 4096], and the
    # IQ4_XS W[4096, 14336] at M = 512
    shapes = {}
    stream = torch.cuda.current_stream().cuda_stream
    for wname, mm in (("q4k_14336x4096_s2", 128), ("q4k_14336x4096_s2", 2048), ("q4k_4096x4096_s2", 128),
                      ("q4k_4096x4096_s2", 512), ("q4k_4096x4096_s2", 2048), ("iq4xs_4096x14336_s3", 512)):
        sfmt, sn, sk, sseed, _ = workloads.WEIGHTS[wname]
        sw = gw if wname == gname else ctx.upload(sfmt, sn, sk, workloads.weight_bytes(wname))
        sx = torch.from_numpy(workloads.activations(sseed, mm, sk)).cuda()
        sa = torch.empty(mm * sk + 2 * mm, dtype=torch.float16, device="cuda")
        sy = torch.empty((mm, sn), dtype=torch.float32, device="cuda")
        ctx.prepare_activations_f16_dev(sx.data_ptr(), mm, sk, sa.data_ptr(), int8=True, stream=stream)

        def skern(i, stream, sw=sw, sa=sa, sy=sy, mm=mm, sk=sk):
            ctx.matmul_f16_dev(sw, sa.data_ptr(), mm, sk, sy.data_ptr(), stream=stream)

        r = GraphRunner(torch, skern, gper, use_graph)
        warm(r, gper)
        t = r.time(gsteps) / gsteps
        sflops = 2.0 * mm * sn * sk
        key = f"{wname.rsplit('_', 1)[0]}_m{mm}"
        shapes[key] = {"kernel_us": round(t * 1e6, 2), "tflops": round(sflops / t / 1e12, 1),
                       "frac": round(sflops / t / 1e12 / F16_MFMA_PEAK_TFLOPS, 4)}
        log(f"gemm {key}: kernel {t * 1e6:.1f} us ({sflops / t / 1e12:.1f} TFLOP/s)")
        if sw is not gw:
            sw.release()
    gemm["shapes"] = shapes
    gw.release()
    return gemm


def cpu_time(fn, seconds, min_reps=3, max_reps=1000):
    """Mean seconds per call of fn() after one warm-up call: at least
    `min_reps` calls, more while under `seconds`."""
    fn()
    reps = 0
    t0 = time.perf_counter()
    while reps < min_reps or (time.perf_counter() - t0 < seconds and reps < max_reps):
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def cpu_part(fmt, wbytes, n, k, x_host, y_gpu, weight_bytes, args, gemv_us, gemm, extra):
    # ---- CPU baseline: the reference's AVX2 path on this host ------------------------
    # The oracle's restatement of columns_q4k_avx2 / columns_iq4xs_avx2 with the
    # reference's column chunking over a pool (src/native/quant.rs:666-744,
    # 1386-1433; src/native/mod.rs:110-152; src/native/pool.rs), at
    # T = the affinity mask's CPU count capped at 16 (the box's CPU share),
    # and at 1 thread; the dense f32 oracle (src/lib.rs:262-318) at the
    # CPU-only matvec.
    import numpy as np

    import oracle
    from magnetar_gpu import workloads

    avail = affinity_threads()
    threads = min(16, avail)
    budget = args.cpu_seconds
    legs = {}

    # config 2 (the headline shape): Q4_K x[1,4096] . W[14336,4096]^T
    got = oracle.baseline_packed_matmul(fmt, wbytes, n, k, x_host, threads)
    err = float(np.max(np.abs(got - y_gpu)))
    t_cpu, reps = cpu_time(lambda: oracle.baseline_packed_matmul(fmt, wbytes, n, k, x_host, threads), budget, 10)
    t_cpu1, _ = cpu_time(lambda: oracle.baseline_packed_matmul(fmt, wbytes, n, k, x_host, 1), budget / 4, 3, 50)
    cpu = {
        "value": round(weight_bytes / t_cpu / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"Q4_K x[1,4096] . W[14336,4096]^T, int8 activations, AVX2 column kernels + "
                   f"pool chunking; 1 warm-up + {reps} timed calls ({t_cpu * 1e3:.3f} ms/call)"),
        "single_thread_GBps": round(weight_bytes / t_cpu1 / 1e9, 2),
        "threads_available": avail,
        "cpu_model": cpu_model(),
        "max_abs_diff_vs_gpu": err,
        "gpu_over_cpu": round(t_cpu / (gemv_us * 1e-6), 1),
    }
    log(f"cpu baseline, config 2 ({threads} of {avail} threads, {cpu_model()}): {t_cpu * 1e3:.3f} ms/call, "
        f"{cpu['value']} GB/s; 1 thread {cpu['single_thread_GBps']} GB/s; max|gpu-cpu| {err:.2e}")

    # config 1: the CPU-only Q4_K matvec x[1,4096] . W[4096,4096]^T, plus the
    # dense f32 oracle on the dequantized weight (ReferenceCpuExecutor's path)
    name1 = "q4k_4096x4096_s0"
    f1, n1, k1, s1, _ = workloads.WEIGHTS[name1]
    w1 = workloads.weight_bytes(name1)
    x1 = workloads.activations(s1, 1, k1)
    b1 = workloads.weight_bytes_per_call(name1)
    t1, r1 = cpu_time(lambda: oracle.baseline_packed_matmul(f1, w1, n1, k1, x1, threads), budget / 4, 10)
    t1s, _ = cpu_time(lambda: oracle.baseline_packed_matmul(f1, w1, n1, k1, x1, 1), budget / 8, 3, 100)
    dense_w = oracle.dequantize(f1, w1, n1, k1)
    td, rd = cpu_time(lambda: oracle.matmul_dense(x1, dense_w, False, True), budget / 4, 2, 20)
    legs["config1_q4k_1x4096x4096"] = {
        "ms_per_call": round(t1 * 1e3, 4), "GBps": round(b1 / t1 / 1e9, 2), "threads": threads,
        "single_thread_ms": round(t1s * 1e3, 4), "dense_f32_oracle_ms": round(td * 1e3, 2),
        "sample": f"{r1} timed calls (AVX2 port), {rd} dense-oracle calls (1 thread, f32 W of 64 MiB)"}
    log(f"cpu baseline, config 1: {t1 * 1e3:.3f} ms/call ({b1 / t1 / 1e9:.2f} GB/s) at {threads} threads, "
        f"{t1s * 1e3:.3f} ms at 1; dense f32 oracle {td * 1e3:.1f} ms")

    # config 3: the prefill GEMM x[512,4096] . W[14336,4096]^T on the CPU path
    name3 = "q4k_14336x4096_s2"
    f3, n3, k3, s3, _ = workloads.WEIGHTS[name3]
    w3 = workloads.weight_bytes(name3)
    x3 = workloads.activations(s3, 512, k3)
    t3, r3 = cpu_time(lambda: oracle.baseline_packed_matmul(f3, w3, n3, k3, x3, threads), budget, 2, 10)
    flops3 = 2.0 * 512 * n3 * k3
    leg3 = {"ms_per_call": round(t3 * 1e3, 2), "TOPs": round(flops3 / t3 / 1e12, 3), "threads": threads,
            "sample": f"the full M=512 call, 1 warm-up + {r3} timed calls"}
    if gemm:
        leg3["gpu_over_cpu"] = round(t3 / (gemm["roofline"]["kernel_us"] * 1e-6), 1)
    legs["config3_q4k_512x14336x4096"] = leg3
    log(f"cpu baseline, config 3 (M=512): {t3 * 1e3:.1f} ms/call, {flops3 / t3 / 1e12:.3f} TOP/s")

    # config 4: IQ4_XS x[1,14336] . W[4096,14336]^T
    name4 = "iq4xs_4096x14336_s3"
    f4, n4, k4, s4, _ = workloads.WEIGHTS[name4]
    w4 = workloads.weight_bytes(name4)
    x4 = workloads.activations(s4, 1, k4)
    b4 = workloads.weight_bytes_per_call(name4)
    t4, r4 = cpu_time(lambda: oracle.baseline_packed_matmul(f4, w4, n4, k4, x4, threads), budget / 2, 10)
    leg4 = {"ms_per_call": round(t4 * 1e3, 4), "GBps": round(b4 / t4 / 1e9, 2), "threads": threads,
            "sample": f"1 warm-up + {r4} timed calls"}
    if "iq4xs_gemv_kernel_us" in extra:
        leg4["gpu_over_cpu"] = round(t4 / (extra["iq4xs_gemv_kernel_us"] * 1e-6), 1)
    legs["config4_iq4xs_1x14336x4096"] = leg4
    log(f"cpu baseline, config 4 (IQ4_XS): {t4 * 1e3:.3f} ms/call, {b4 / t4 / 1e9:.2f} GB/s")
    cpu["legs"] = legs
    return cpu


def emit(args, value, steps, warmup, ms_per_step, n, k, weight_bytes, use_graph, step_runner, achieved, kernel_us,
         cpu, gemm, extra):
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "Q4_K decode GEMV x[1,4096] . W[14336,4096]^T (Llama-3-8B FFN up), seed 1",
            "m": 1, "n": n, "k": k, "weight_bytes": weight_bytes, "weight_copies": args.copies,
            "launch": "hip_graph" if (use_graph and step_runner.graph is not None) else "eager",
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": recorded_traffic("gemv_q4k_m1_fused"),
            "traffic_unit": "HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "algorithmic_bytes": weight_bytes + 4 * k + 4 * n, "kernel_us": round(kernel_us, 3),
            "kernel": "gemv_wave_int8_kernel<Q4_K, 1, fused> (one super-block per wave, 16 waves per 64 rows): int8 quantization of x in LDS + Q4_K GEMV, one launch",
        },
        "cpu_baseline": cpu,
        "gemm": gemm,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
