#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-linear hot path (BASELINE.json's metric, one GPU).

Headline (`value`): config 2 of BASELINE.json -- FP8 e4m3 decode linear, M=1, K=1024, N=3584,
bf16 activations in and bf16 out through the FP8 boundary (the exported Cast -> MatMul -> Cast
chain, fused into one kernel) -- as HBM GB/s of algorithmic bytes.  One step = one call over one
activation row.  80 weight copies (294 MB > the 256 MB MALL) are rotated so every step streams its
weight from HBM.  Steps are captured once into a HIP graph through the library's own capture API
(fhip_capture_*) and the graph is replayed; the timed region is bracketed by a device
synchronisation on both sides.

`roofline`: the headline kernel's algorithmic bytes / its average launch duration.  Each timed step is
exactly one launch of that kernel, so the average duration is the timed region (HIP events on the
kernel's stream) over the launch count; per-launch event pairs from a separate eager pass are reported
beside it (they include the event overhead).  `traffic` is the HBM bytes per launch measured by
rocprofv3 FETCH_SIZE / WRITE_SIZE, calibrated on a copy kernel (profiles/fp8_gemv_decode_m1.*).
`cpu_baseline`: the reference's own x86 FP8 linear (oracle/_ref, built from the Feather sources)
on the host, M=1 with its prepared (BF16-packed) weight, for a bounded ~10 s sample.
`configs`: the other BASELINE.json configs (C1, C2 M=4/16, C3, C4, C5), same method.  C1 and C4 rotate copies
of their operands past the 256 MB MALL, so their ms_per_step reads HBM; the single-copy figure is beside it.
`measured_ceilings`: what the chip sustains beside the published peaks -- the FP8 MFMA rate with the C3
operand codes (and with zero codes) in the registers, and the L2 -> LDS staging rate (ceilings()).
"""
import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "FP8/INT8 GEMM TOPS (% MFMA peak) + decode GEMV HBM GB/s (% peak), 1 GPU"
# library backend name of the headline call -> the kernel it launches (as rocprofv3 names it)
HEADLINE_KERNELS = {"fp8_gemv_m1": "fp8_gemv1_kernel<false, 1, 2, 2, true, true>"}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=4000)
    p.add_argument("--warmup", type=int, default=400)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only-headline", action="store_true")
    p.add_argument("--copies", type=int, default=80,
                   help="weight copies the headline rotates through (80 x 3.67 MB = 294 MB > the 256 MB MALL)")
    p.add_argument("--trace-headline", action="store_true",
                   help="headline only, graph-replayed launches only (no eager event pairs or dispatch reference "
                        "points): the run rocprofv3 traces for the headline kernel's per-dispatch duration")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--configs", default="", help="comma list of extra configs to run (C1..C5; default all; I8L: opt-in INT8 linear at larger M)")
    return p.parse_args()


def fp8_pow2_scale(amax, e5):
    maxf = 57344.0 if e5 else 448.0
    return 1.0 if not amax > 0 else float(2.0 ** math.ceil(math.log2(amax / maxf)))


class Bench:
    def __init__(self, args):
        import torch
        from infer_amd import _lib as L
        from infer_amd.runtime import Context
        self.torch, self.L = torch, L
        self.ctx = Context(0)
        self.s = self.ctx.stream
        self.gen = torch.Generator(device="cuda")
        self.args = args

    # -- data ---------------------------------------------------------------------------------
    def randn(self, shape, seed, std=1.0):
        self.gen.manual_seed(seed)
        return self.torch.randn(shape, generator=self.gen, device="cuda", dtype=self.torch.float32) * std

    def to_fp8(self, x, dtype):
        """fp32 device tensor -> (codes, pow2 scale) with the library's own Cast."""
        t = self.torch
        s = fp8_pow2_scale(float(x.abs().max()), dtype == self.L.FP8E5M2)
        codes = t.empty(x.shape, dtype=t.uint8, device="cuda")
        self.ctx.cast(x, self.L.FP32, 1.0, codes, dtype, s)
        return codes, s

    def decode(self, codes, dtype, scale):
        out = self.torch.empty(codes.shape, dtype=self.torch.float32, device="cuda")
        self.ctx.cast(codes, dtype, scale, out, self.L.FP32, 1.0)
        return out

    # -- timing ---------------------------------------------------------------------------------
    def graph_time(self, steps, reps, warm=3, eager_warm=True):
        """steps: callables, each enqueues one step on ctx.stream.  Returns ms per step."""
        t, ctx = self.torch, self.ctx
        with t.cuda.stream(self.s):
            if eager_warm:
                for f in steps:  # eager warm-up grows workspaces before capture
                    f()
            ctx.synchronize()
            ctx.capture_begin()
            for f in steps:
                f()
            g = ctx.capture_end()
            for _ in range(warm):
                ctx.graph_launch(g)
            t.cuda.synchronize()
            e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            wall = time.perf_counter()
            e0.record(self.s)
            for _ in range(reps):
                ctx.graph_launch(g)
            e1.record(self.s)
            t.cuda.synchronize()
            wall = time.perf_counter() - wall
        ctx.graph_destroy(g)
        ms = e0.elapsed_time(e1)
        return ms / (reps * len(steps)), wall

    def kernel_time(self, step, n):
        """Mean duration of one launch from event pairs around each launch (eager, same stream)."""
        t = self.torch
        evs = [(t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)) for _ in range(n)]
        with t.cuda.stream(self.s):
            step(0)
            t.cuda.synchronize()
            for i, (a, b) in enumerate(evs):
                a.record(self.s)
                step(i)
                b.record(self.s)
            t.cuda.synchronize()
        d = [a.elapsed_time(b) for a, b in evs]
        return statistics.mean(d), statistics.median(d)


def headline(b, args):
    t, L, ctx = b.torch, b.L, b.ctx
    k, n, copies = 1024, 3584, args.copies
    w = b.randn((k, n), 0xFEA70002, 0.02)                  # MatMul weight [K,N] (exporter layout)
    w_codes, sw = b.to_fp8(w, L.FP8E4M3)
    x = b.randn((1, k), 0xFEA70002 + 1)
    xb = x.to(t.bfloat16)
    s_in = fp8_pow2_scale(float(xb.float().abs().max()), False)
    xc = t.empty((1, k), dtype=t.uint8, device="cuda")
    ctx.cast(xb, L.BF16, 1.0, xc, L.FP8E4M3, s_in)
    y = b.decode(xc, L.FP8E4M3, s_in) @ b.decode(w_codes, L.FP8E4M3, sw)
    s_out = fp8_pow2_scale(float(y.abs().max()), False)
    srcs = [w_codes.clone() for _ in range(copies)]
    weights = [ctx.prepare_weight(s_, L.FP8E4M3, k, n, L.LAYOUT_KN, version=1) for s_ in srcs]
    out = t.empty((1, n), dtype=t.bfloat16, device="cuda")

    def step(i):
        ctx.fp8_linear(xb, L.BF16, s_in, 1, weights[i % copies], sw, out, L.BF16, s_out)

    ctx.synchronize()
    backend = None
    with t.cuda.stream(b.s):
        step(0)  # the one eager call: names the kernel path (the GEMV needs no workspace to grow)
        backend = ctx.last_backend()
    # exactly args.steps timed steps: replays of one graph of `per_graph` launches (the largest divisor of
    # the step count up to 400, so short runs are not rounded up)
    total = max(1, args.steps)
    per_graph = max(d for d in range(1, min(400, total) + 1) if total % d == 0)
    reps = total // per_graph
    steps = [(lambda i=i: step(i)) for i in range(per_graph)]
    with t.cuda.stream(b.s):
        for i in range(args.warmup):  # the untimed warm-up steps
            step(i)
    # one untimed replay uploads the graph before the timed replays
    ms, wall = b.graph_time(steps, reps, warm=1, eager_warm=False)
    kmean, kmed = b.kernel_time(step, 800) if not args.trace_headline else (None, None)
    bytes_step = k * n + k * 2 + n * 2
    res = {
        "ms_per_step": ms, "steps": reps * per_graph, "wall_s": wall, "bytes": bytes_step,
        "value": bytes_step / (ms * 1e-3) / 1e9, "kernel_ms": kmean, "kernel_ms_median": kmed,
        "backend": backend, "backend_kernel": HEADLINE_KERNELS.get(backend),
    }
    for wt in weights:
        wt.release()
    return res


def dispatch_floor(b, nbytes=3670016, copies=80, per_graph=400, reps=5):
    """Reference points for a single dispatch of the headline's size, not this library's code: torch's
    device copy of the same 3.67 MB weight (it also writes 3.67 MB) from rotated buffers, and an empty
    kernel (torch.cuda._sleep(0)), each one launch per graph node of a replayed torch CUDA graph."""
    t = b.torch
    out = {}
    try:
        srcs = [t.empty(nbytes, dtype=t.uint8, device="cuda") for _ in range(copies)]
        dst = t.empty(nbytes, dtype=t.uint8, device="cuda")
        for name, fn in (("copy_3670016B_us", lambda i: dst.copy_(srcs[i % copies])),
                         ("empty_kernel_us", lambda i: t.cuda._sleep(0))):
            s = t.cuda.Stream()
            s.wait_stream(t.cuda.current_stream())
            with t.cuda.stream(s):
                for i in range(3):
                    fn(i)
            t.cuda.current_stream().wait_stream(s)
            g = t.cuda.CUDAGraph()
            with t.cuda.graph(g):
                for i in range(per_graph):
                    fn(i)
            for _ in range(3):
                g.replay()
            t.cuda.synchronize()
            e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            t.cuda.synchronize()
            out[name] = e0.elapsed_time(e1) * 1e3 / (reps * per_graph)
            del g
    except Exception as e:  # reference point only: report, do not fail the bench
        out["error"] = repr(e)[:200]
    return out


def cpu_headline(args):
    """Reference x86 FP8 linear (prepared BF16-packed RHS), M=1, K=1024, N=3584, on host cores."""
    import ctypes
    import numpy as np
    from oracle import pyoracle as po
    if not po.ref_available():
        return None
    R = po.ref()
    r = np.random.default_rng(0xFEA70002)
    w = (r.standard_normal((1024, 3584), dtype=np.float32) * np.float32(0.02))
    sw = fp8_pow2_scale(float(np.abs(w).max()), False)
    wc = po.fp8_encode(po.FP8E4M3, w / np.float32(sw))
    x = r.standard_normal((1, 1024), dtype=np.float32)
    s_in = fp8_pow2_scale(float(np.abs(x).max()), False)
    xc = po.fp8_encode(po.FP8E4M3, x / np.float32(s_in))
    out = np.empty((1, 3584), np.uint8)
    h = R.ref_fp8_packed_create(po.FP8E4M3, po._ptr(wc), 0, 1024, 3584)
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    calls = 0
    while time.perf_counter() < t_end or calls < 20:
        t0 = time.perf_counter()
        rc = R.ref_fp8_packed_compute(h, po._ptr(xc), s_in, sw, 1, po._ptr(out), 1.0)
        times.append(time.perf_counter() - t0)
        calls += 1
        assert rc == 0
    R.ref_fp8_packed_destroy(h)
    med = statistics.median(times)
    threads = min(4, R.ref_max_threads())
    bytes_step = 1024 * 3584 + 1024 * 2 + 3584 * 2
    return {
        "value": bytes_step / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "reference",
        "sample": f"{calls} calls (~{args.cpu_seconds:.0f} s) of Feather x86 ComputeLinearRowMajorX86Fp8PackedRhs, "
                  f"M=1 K=1024 N=3584 e4m3, median {med * 1e3:.3f} ms/call; the two memory-bound Cast nodes "
                  f"(1024 + 3584 elements) are not included; host nproc={os.cpu_count()}",
    }


def _time_calls(fn, seconds, min_calls=5):
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_calls:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_configs(args):
    """CPU baselines of the other configs on the host cores, each a bounded sample (~3 s).
    With oracle/_ref present every config runs the reference's own x86 kernels, with its thread policy:
    INT8 Gemm 1 thread (x86/int8.cc:514-572), INT8 conv every OpenMP thread (int8.cc:2331-2334), FP8 linear
    and BF16 argmax min(4, OpenMP) workers.  Without it, C1 and C4 fall back to the C restatement of the
    Common kernels (oracle/liboracle.so, "kind": "port")."""
    import numpy as np
    from oracle import pyoracle as po
    res = {}
    budget = max(1.0, args.cpu_seconds / 3.0)
    r = np.random.default_rng(0xFEA70010)
    L = po.lib()
    all_threads = L.fo_set_threads(0)
    have_ref = po.ref_available()
    # C1: QuantizeLinear -> INT8 Gemm (transB) -> DequantizeLinear is dominated by the Gemm; 1 thread
    m, k, n = 128, 1024, 1024
    a = r.integers(-127, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    ws = r.uniform(1e-3, 1e-2, n).astype(np.float32)
    bias = r.integers(-20000, 20000, n).astype(np.int32)
    if have_ref:
        R = po.ref()
        R.ref_set_threads(1)
        h = R.ref_i8_gemm_create(po._ptr(a), 0.03, 0, m, k, po._ptr(w), po._ptr(ws), n, n, po._ptr(bias), 1.0, 1.0,
                                 0.05, 0)
        med, calls = _time_calls(lambda: R.ref_i8_gemm_compute(h), budget)
        R.ref_i8_gemm_destroy(h)
        res["C1"] = {"value": 2.0 * m * k * n / med / 1e12, "unit": "TOPS", "cores": 1, "kind": "reference",
                     "sample": f"{calls} calls of Feather x86 GemmKernel<X86, INT8> (int8.cc:514-572), "
                               f"128x1024x1024 transB, median {med * 1e3:.1f} ms; the Common QuantizeLinear and "
                               f"DequantizeLinear nodes are not included"}
    else:
        L.fo_set_threads(1)
        med, calls = _time_calls(lambda: po.i8_linear(po.I8_GEMM, a, 0.03, 0, w, True, ws, None, bias, po.BIAS_VECTOR,
                                                      1.0, 1.0, 0.05, 0), budget)
        res["C1"] = {"value": 2.0 * m * k * n / med / 1e12, "unit": "TOPS", "cores": 1, "kind": "port",
                     "sample": f"{calls} calls of the INT8 Gemm 128x1024x1024 restated from the Common kernel, "
                               f"median {med * 1e3:.2f} ms"}
    # C4: INT8 conv 3x3 s2 p1, all threads
    L.fo_set_threads(all_threads)
    x = r.integers(-128, 128, (1, 64, 160, 160)).astype(np.int8)
    wc = r.integers(-127, 128, (128, 64, 3, 3)).astype(np.int8)
    wcs = r.uniform(1e-3, 1e-2, 128).astype(np.float32)
    cb = r.integers(-5000, 5000, 128).astype(np.int32)
    if have_ref:
        R.ref_set_threads(all_threads)
        h = R.ref_i8_conv2d_create(po._ptr(x), 1, 64, 160, 160, 0, 0.05, 0, po._ptr(wc), 128, 3, 3, 1, po._ptr(wcs),
                                   po._ptr(cb), 2, 2, 1, 1, 1, 1, 80, 80, 0.5, 0)
        R.ref_i8_conv2d_compute(h)  # packs the weights once, as Prepare-time caching does
        med, calls = _time_calls(lambda: R.ref_i8_conv2d_compute(h), budget)
        R.ref_i8_conv2d_destroy(h)
        path = "VNNI" if R.ref_has_avx_vnni() else "AVX2 maddubs"
        res["C4"] = {"value": 943718400 / med / 1e12, "unit": "TOPS", "cores": all_threads, "kind": "reference",
                     "sample": f"{calls} calls of Feather x86 Conv2DKernel<X86, INT8> ({path} path, int8.cc:684-2346), "
                               f"[1,64,160,160] x [128,64,3,3] s2 p1, median {med * 1e3:.2f} ms"}
    else:
        med, calls = _time_calls(lambda: po.i8_conv2d(x, 0.05, 0, wc, wcs, cb, 2, 1, 0.5, 0), budget)
        res["C4"] = {"value": 943718400 / med / 1e12, "unit": "TOPS", "cores": all_threads, "kind": "port",
                     "sample": f"{calls} calls of the INT8 Conv2D [1,64,160,160] x [128,64,3,3] s2 p1 restated from "
                               f"the Common kernel, median {med * 1e3:.1f} ms"}
    if po.ref_available():
        R = po.ref()
        threads = min(4, R.ref_max_threads())
        # C3: x86 FP8 linear (direct kernel) on a 32-row sample of the up-projection, e5m2
        rows, k3, n3 = 32, 1024, 3584
        a3 = po.fp8_encode(po.FP8E5M2, r.standard_normal((rows, k3)).astype(np.float32))
        w3 = po.fp8_encode(po.FP8E5M2, (r.standard_normal((n3, k3)) * 0.02 * 2 ** 10).astype(np.float32))
        y3 = np.empty((rows, n3), np.uint8)
        med, calls = _time_calls(lambda: R.ref_fp8_linear(po.FP8E5M2, po._ptr(a3), 1.0, po._ptr(w3), 2.0 ** -10, 1,
                                                          None, 1.0, 0, 1.0, 1.0, rows, k3, n3, po._ptr(y3), 1.0),
                                 budget)
        res["C3"] = {"value": 2.0 * rows * k3 * n3 / med / 1e12, "unit": "TFLOP/s", "cores": threads,
                     "kind": "reference",
                     "sample": f"{calls} calls of Feather x86 ComputeLinearRowMajorX86Fp8TransposedRhs on {rows} of "
                               f"the 4096 up-projection rows, median {med * 1e3:.2f} ms"}
        # C5: x86 BF16 LM-head argmax, M=1 (packed transposed RHS, prepared once)
        v5, k5 = 151936, 1024
        w5 = po.bf16_encode((r.standard_normal((v5, k5), dtype=np.float32) * np.float32(0.02)))
        a5 = po.bf16_encode(r.standard_normal(k5).astype(np.float32))
        h = R.ref_bf16_argmax_create(po._ptr(w5), k5, v5)
        tok = ctypes.c_int64()
        med, calls = _time_calls(lambda: R.ref_bf16_argmax_compute(h, po._ptr(a5), ctypes.byref(tok)), budget)
        R.ref_bf16_argmax_destroy(h)
        res["C5"] = {"value": (v5 * k5 * 2 + k5 * 2 + 8) / med / 1e9, "unit": "GB/s", "cores": threads,
                     "kind": "reference",
                     "sample": f"{calls} calls of Feather x86 ComputeLinearRowMajorX86Bf16PackedTransposedRhsArgmax, "
                               f"M=1 K=1024 V=151936, median {med * 1e3:.1f} ms"}
    return res


def vendor_fp8_gemm_us(b, m, k, n):
    """Reference point only (not this library): the vendor FP8 GEMM, torch._scaled_mm -> hipBLASLt, e5m2 x e5m2
    -> bf16 on the C3 up- and down-projection shapes, random operands, eager launches timed with events."""
    t = b.torch
    out = {}
    try:
        for name, (mm, kk, nn) in (("up", (m, k, n)), ("down", (m, n, k))):
            a = (t.randn(mm, kk, device="cuda") * 0.5).to(t.float8_e5m2)
            w = (t.randn(nn, kk, device="cuda") * 0.5).to(t.float8_e5m2)
            one = t.tensor(1.0, device="cuda")

            def f():
                return t._scaled_mm(a, w.t(), scale_a=one, scale_b=one, out_dtype=t.bfloat16)
            for _ in range(20):
                f()
            t.cuda.synchronize()
            e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(100):
                f()
            e1.record()
            t.cuda.synchronize()
            us = e0.elapsed_time(e1) * 10.0
            out[name + "_us"] = us
            out[name + "_TFLOP/s"] = 2.0 * mm * nn * kk / us / 1e6
    except Exception as e:  # absent on some builds: report, do not fail the bench
        out["error"] = repr(e)[:200]
    return out


def extra_configs(b, args):
    t, L, ctx = b.torch, b.L, b.ctx
    res = {}
    chosen = set(args.configs.split(",")) if args.configs else None

    def want(tag):
        return chosen is None or tag in chosen

    if want("C2"):
        # C2 M=4, 16
        k, n, copies = 1024, 3584, 80
        w_codes, sw = b.to_fp8(b.randn((k, n), 0xFEA70002, 0.02), L.FP8E4M3)
        srcs = [w_codes.clone() for _ in range(copies)]
        weights = [ctx.prepare_weight(s_, L.FP8E4M3, k, n, L.LAYOUT_KN, version=2) for s_ in srcs]
        for m in (4, 16):
            xb = b.randn((m, k), 0xFEA70002 + m).to(t.bfloat16)
            out = t.empty((m, n), dtype=t.bfloat16, device="cuda")

            def step(i, xb=xb, out=out, m=m):
                ctx.fp8_linear(xb, L.BF16, 0.0078125, m, weights[i % copies], sw, out, L.BF16, 0.03125)
            ms, _ = b.graph_time([(lambda i=i: step(i)) for i in range(200)], 5)
            km, _ = b.kernel_time(step, 200)
            by = k * n + m * k * 2 + m * n * 2
            res[f"C2_fp8_decode_M{m}"] = {"ms_per_step": ms, "GB/s": by / ms / 1e6, "hbm_frac": by / ms / 1e6 / HBM_PEAK_GBS,
                                          "kernel_ms_event_pairs": km}
        for wt in weights:
            wt.release()
        del srcs

    if want("C3"):
        # C3 FP8 e5m2 prefill: up-proj [4096,1024]x[1024->3584], down-proj [4096,3584]x[3584->1024]
        m, k, n = 4096, 1024, 3584
        E5 = L.FP8E5M2
        a_codes, sa = b.to_fp8(b.randn((m, k), 0xFEA70003), E5)
        wu_codes, su = b.to_fp8(b.randn((n, k), 0xFEA70003 + 1, 0.02), E5)
        wd_codes, sd = b.to_fp8(b.randn((k, n), 0xFEA70003 + 2, 0.02), E5)
        wu = ctx.prepare_weight(wu_codes, E5, k, n, L.LAYOUT_NK, version=3)
        wd = ctx.prepare_weight(wd_codes, E5, n, k, L.LAYOUT_NK, version=3)
        mid = t.empty((m, n), dtype=t.uint8, device="cuda")
        out = t.empty((m, k), dtype=t.bfloat16, device="cuda")
        s_mid, s_o = 0.125, 0.25

        def up(i=0):
            ctx.fp8_linear(a_codes, E5, sa, m, wu, su, mid, E5, s_mid)

        def down(i=0):
            ctx.fp8_linear(mid, E5, s_mid, m, wd, sd, out, L.BF16, s_o)
        # MFMA-bound: enough warm-up replays for the clocks to settle after the bandwidth-bound configs
        ms, _ = b.graph_time([up, down] * 10, 50, warm=20)
        ku, _ = b.kernel_time(up, 50)
        kd, _ = b.kernel_time(down, 50)
        fl = 2.0 * m * k * n
        vendor = vendor_fp8_gemm_us(b, m, k, n)
        res["C3_fp8e5m2_prefill"] = {
            "ms_per_gemm": ms, "TFLOP/s": fl / ms / 1e9, "mfma_frac": fl / ms / 1e9 / FP8_PEAK_TFLOPS,
            "up_kernel_ms_event_pairs": ku, "up_TFLOP/s_event_pairs": fl / ku / 1e9,
            "down_kernel_ms_event_pairs": kd, "down_TFLOP/s_event_pairs": fl / kd / 1e9,
            "reference_point_hipblaslt": vendor,
            "backend": ctx.last_backend()}
        wu.release()
        wd.release()

    if want("C1"):
        # C1 INT8 linear chain: QuantizeLinear(fp32) -> Gemm INT8 (transB) -> DequantizeLinear(fp32)
        m, k, n = 128, 1024, 1024
        x = b.randn((m, k), 0xFEA70001)
        s_x = float(x.abs().max()) / 127.0
        b.gen.manual_seed(0xFEA70001 + 1)
        wq = t.randint(-127, 128, (n, k), generator=b.gen, device="cuda", dtype=t.int8)
        s_w = (t.rand(n, generator=b.gen, device="cuda") * 9e-3 + 1e-3).cpu().numpy()
        bias = t.randint(-20000, 20000, (n,), generator=b.gen, device="cuda", dtype=t.int32)
        w8 = ctx.prepare_weight(wq, L.INT8, k, n, L.LAYOUT_NK, scales=s_w, version=4)
        xq = t.empty((m, k), dtype=t.int8, device="cuda")
        yq = t.empty((m, n), dtype=t.int8, device="cuda")
        y = t.empty((m, n), dtype=t.float32, device="cuda")
        s_y = 0.05

        def c1(i=0):  # QuantizeLinear, then Gemm with the DequantizeLinear fused into its epilogue
            ctx.quantize_linear(x, L.FP32, [s_x], [0], xq)
            ctx.i8_linear_ex(L.I8_GEMM, xq, s_x, 0, m, w8, y, L.FP32, s_y, 0, dq_scale=s_y, dq_zp=0, bias=bias,
                             bias_kind=L.BIAS_VECTOR, bias_abs_max=20000)

        def c1_unfused(i=0):  # the three nodes as three launches
            ctx.quantize_linear(x, L.FP32, [s_x], [0], xq)
            ctx.i8_linear(L.I8_GEMM, xq, s_x, 0, m, w8, yq, s_y, 0, bias=bias, bias_kind=L.BIAS_VECTOR, bias_abs_max=20000)
            ctx.dequantize_linear(yq, [s_y], [0], y, L.FP32)

        def c1_gemm(i=0):
            ctx.i8_linear(L.I8_GEMM, xq, s_x, 0, m, w8, yq, s_y, 0, bias=bias, bias_kind=L.BIAS_VECTOR, bias_abs_max=20000)
        # Rotated copies of the activation and the prepared weight (200 x 1.5 MB = 300 MB > the 256 MB MALL), so
        # every step reads its operands from HBM; the single-copy figure (operands cache-resident) beside it.
        copies = 200
        xs = [x.clone() for _ in range(copies)]
        wsrc = [wq.clone() for _ in range(copies)]  # kept alive until the preparation kernels have read them
        ws = [ctx.prepare_weight(src, L.INT8, k, n, L.LAYOUT_NK, scales=s_w, version=4) for src in wsrc]
        ctx.synchronize()
        del wsrc

        def c1_rot(i, xi, wi):
            ctx.quantize_linear(xi, L.FP32, [s_x], [0], xq)
            ctx.i8_linear_ex(L.I8_GEMM, xq, s_x, 0, m, wi, y, L.FP32, s_y, 0, dq_scale=s_y, dq_zp=0, bias=bias,
                             bias_kind=L.BIAS_VECTOR, bias_abs_max=20000)
        ms, _ = b.graph_time([lambda i=0, xi=xi, wi=wi: c1_rot(i, xi, wi) for xi, wi in zip(xs, ws)], 3)
        ms_res, _ = b.graph_time([c1] * 50, 10)
        ms_unfused, _ = b.graph_time([c1_unfused] * 50, 10)
        kg, _ = b.kernel_time(c1_gemm, 200)
        ops = 2.0 * m * k * n
        res["C1_int8_linear_chain"] = {"ms_per_step": ms, "ms_per_step_cache_resident": ms_res,
                                       "ms_per_step_three_launches_cache_resident": ms_unfused,
                                       "TOPS": ops / ms / 1e9, "GB/s": 2101248 / ms / 1e6,
                                       "int8_frac": ops / ms / 1e9 / INT8_PEAK_TOPS,
                                       "operands": f"{copies} rotated copies (300 MB > MALL)",
                                       "gemm_kernel_ms_event_pairs": kg}
        for wi in ws:
            wi.release()
        del xs
        w8.release()

    if want("C4"):
        # C4 INT8 conv 3x3 s2 p1 [1,64,160,160] -> [1,128,80,80]
        b.gen.manual_seed(0xFEA70004)
        xin = t.randint(-128, 128, (1, 64, 160, 160), generator=b.gen, device="cuda", dtype=t.int8)
        wc = t.randint(-127, 128, (128, 64, 3, 3), generator=b.gen, device="cuda", dtype=t.int8)
        sc = (t.rand(128, generator=b.gen, device="cuda") * 9e-3 + 1e-3).cpu().numpy()
        cb = t.randint(-20000, 20000, (128,), generator=b.gen, device="cuda", dtype=t.int32)
        wcp = ctx.prepare_conv_weight(wc, sc, version=5)
        yc = t.empty((1, 128, 80, 80), dtype=t.int8, device="cuda")

        def c4(i=0):
            ctx.i8_conv2d(xin, L.NCHW, 0.0078125, 0, wcp, yc, 0.25, 0, stride=(2, 2), pad=(1, 1), bias=cb,
                          bias_abs_max=20000)
        # 170 rotated input copies (272 MB > the 256 MB MALL): every step reads its input from HBM
        copies = 170
        xins = [xin.clone() for _ in range(copies)]

        def c4_rot(i, xi):
            ctx.i8_conv2d(xi, L.NCHW, 0.0078125, 0, wcp, yc, 0.25, 0, stride=(2, 2), pad=(1, 1), bias=cb,
                          bias_abs_max=20000)
        ms, _ = b.graph_time([lambda i=0, xi=xi: c4_rot(i, xi) for xi in xins], 3)
        ms_res, _ = b.graph_time([c4] * 50, 10)
        kc, _ = b.kernel_time(c4, 100)
        ops = 943718400.0
        res["C4_int8_conv3x3s2"] = {"ms_per_step": ms, "ms_per_step_cache_resident": ms_res,
                                    "TOPS": ops / ms / 1e9, "GB/s": 2531840 / ms / 1e6,
                                    "int8_frac": ops / ms / 1e9 / INT8_PEAK_TOPS,
                                    "hbm_frac": 2531840 / ms / 1e6 / HBM_PEAK_GBS,
                                    "operands": f"{copies} rotated input copies (272 MB > MALL)", "kernel_ms_event_pairs": kc}
        del xins
        wcp.release()

    if want("C5"):
        # C5 BF16 LM head + argmax, V=151936 (311 MB > MALL)
        k, v = 1024, 151936
        wh = (b.randn((v, k), 0xFEA70005, 0.02)).to(t.bfloat16)
        for m in (1, 8):
            a = b.randn((m, k), 0xFEA70005 + m).to(t.bfloat16)
            tok = t.empty(m, dtype=t.int64, device="cuda")

            def c5(i=0, a=a, tok=tok):
                ctx.bf16_gemv_argmax(a, wh, tok)
            ms, _ = b.graph_time([c5] * 20, 10)
            km, _ = b.kernel_time(c5, 50)
            by = v * k * 2 + m * k * 2 + m * 8
            res[f"C5_bf16_argmax_M{m}"] = {"ms_per_step": ms, "GB/s": by / ms / 1e6, "hbm_frac": by / ms / 1e6 / HBM_PEAK_GBS,
                                           "kernel_ms_event_pairs": km}

    if chosen is not None and "I8L" in chosen:
        # Opt-in (not a BASELINE config): the INT8 linear at larger M, where fhip_i8_linear runs the MFMA tile
        # GEMM; FC, per-channel weight scales, INT8 output.  Operands stay resident (MFMA-bound shapes).
        for m, k, n in ((4096, 4096, 4096), (4096, 18944, 3584), (1024, 4096, 4096), (4096, 1024, 3584)):
            b.gen.manual_seed(0xFEA7000A + m + k + n)
            a8 = t.randint(-128, 128, (m, k), generator=b.gen, device="cuda", dtype=t.int8)
            w8 = t.randint(-127, 128, (n, k), generator=b.gen, device="cuda", dtype=t.int8)
            s_w = (t.rand(n, generator=b.gen, device="cuda") * 9e-3 + 1e-3).cpu().numpy()
            wp = ctx.prepare_weight(w8, L.INT8, k, n, L.LAYOUT_NK, scales=s_w, version=10)
            o8 = t.empty((m, n), dtype=t.int8, device="cuda")

            def i8l(i=0, a8=a8, wp=wp, o8=o8, m=m):
                ctx.i8_linear(L.I8_FC, a8, 0.01, 0, m, wp, o8, 0.5, 0)
            ms, _ = b.graph_time([i8l] * 10, 5)
            tops = 2.0 * m * n * k / ms / 1e9
            res[f"I8L_int8_fc_{m}x{k}x{n}"] = {"ms_per_step": ms, "TOPS": tops, "mfma_frac": tops / INT8_PEAK_TOPS,
                                               "backend": ctx.last_backend()}
            wp.release()
            del a8, w8, o8

    return res


def ceilings(b):
    """Measured ceilings beside the published peaks (bench_ceilings.hip beside this file, not part of the operator
    library): the sustained FP8 MFMA rate with the C3 activation codes, and with all-zero codes, in the
    operand registers (MFMA power, and so the sustained clock, depends on the operand bits), and the
    L2 -> LDS rate of the GEMM's operand staging path over an L2-resident 2 MB buffer."""
    t, L = b.torch, b.L
    lib = ctypes.CDLL(os.path.join(ROOT, "bench_ceilings.so"))
    lib.fhipc_mfma_fp8_rate.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_float)]
    lib.fhipc_l2_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    codes, _ = b.to_fp8(b.randn((4096, 1024), 0xFEA70003), L.FP8E5M2)  # the C3 activations
    zeros = t.zeros(1 << 16, dtype=t.uint8, device="cuda")
    buf = t.ones(2 << 20, dtype=t.uint8, device="cuda")
    t.cuda.synchronize()
    out = {}
    for name, src in (("mfma_fp8_tflops_c3_operands", codes), ("mfma_fp8_tflops_zero_operands", zeros)):
        v = ctypes.c_float(0.0)
        rc = lib.fhipc_mfma_fp8_rate(src.data_ptr(), src.numel(), 1, 4000, ctypes.byref(v))
        out[name] = round(v.value, 1) if rc == 0 else f"error {rc}"
    v = ctypes.c_float(0.0)
    rc = lib.fhipc_l2_stream(buf.data_ptr(), buf.numel(), 400, ctypes.byref(v))
    out["l2_to_lds_tbs"] = round(v.value, 2) if rc == 0 else f"error {rc}"
    out["note"] = ("mfma: one 512-thread block per CU, 4 independent v_mfma_scale_f32_32x32x64_f8f6f4 chains; "
                   "l2: 16-byte buffer_load...lds, one 512-thread block per CU, 2 MB L2-resident buffer")
    return out


def traced_duration(kernel):
    """The committed rocprofv3 kernel-trace statistics of the headline kernel's timed launches
    (profiles/fp8_gemv_decode_m1.trace.json), or None when that summary is of another kernel."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "fp8_gemv_decode_m1.trace.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel:
        return None
    return {"avg_us": t["avg_ns"] / 1e3, "median_us": t["median_ns"] / 1e3, "min_us": t["min_ns"] / 1e3,
            "launches": t["launches"], "source": "profiles/fp8_gemv_decode_m1.trace.json"}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/fp8_gemv_decode_m1.traffic.json), or None when that summary is of another kernel."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "fp8_gemv_decode_m1.traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t["bytes_per_launch"] if t.get("kernel") == kernel else None


def main():
    args = parse()
    if args.trace_headline:
        args.only_headline, args.no_cpu = True, True
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    b = Bench(args)
    h = headline(b, args)
    line = {
        "metric": METRIC,
        "value": round(h["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": h["steps"],
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, power-of-two FP8 scales)",
        "config": {
            "workload": "C2: FP8 e4m3 decode linear M=1 K=1024 N=3584, bf16 in -> Cast(fp8) -> MatMul -> "
                        "Cast(bf16) fused in one kernel; 80 rotated weight copies (294 MB)",
            "kernel": h["backend"], "graph_replayed": True,
        },
        # Each timed step is exactly one launch of the headline kernel, so the kernel's average launch
        # duration is the timed region over the launch count (events on the kernel's stream).
        "roofline": {
            "bound": "hbm", "achieved": round(h["bytes"] / h["ms_per_step"] / 1e6, 2), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(h["bytes"] / h["ms_per_step"] / 1e6 / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(h["backend_kernel"]), "kernel_ms": h["ms_per_step"],
            "kernel_ms_event_pairs": h["kernel_ms"], "kernel_ms_event_pairs_median": h["kernel_ms_median"],
        },
        "cpu_baseline": None,
    }
    tr = traced_duration(h["backend_kernel"])
    if tr is not None:
        # the same launches timed one by one by rocprofv3's kernel trace (each dispatch's own begin/end
        # timestamps, which the profiler takes with the pipeline between dispatches drained)
        tr["frac_at_avg"] = round(h["bytes"] / (tr["avg_us"] * 1e3) / HBM_PEAK_GBS, 4)
        tr["frac_at_median"] = round(h["bytes"] / (tr["median_us"] * 1e3) / HBM_PEAK_GBS, 4)
        line["roofline"]["rocprof_trace"] = tr
    if not args.trace_headline:
        # What one dispatch of this size costs on this chip whatever the kernel does: an empty kernel, and a
        # device copy of the same weight bytes, each replayed the same way.  The headline kernel's time splits
        # into that launch floor and its own excess.
        fl = dispatch_floor(b)
        line["dispatch_reference_points"] = fl
        if "empty_kernel_us" in fl:
            kus = h["ms_per_step"] * 1e3
            line["roofline"]["floor"] = {
                "empty_kernel_us": round(fl["empty_kernel_us"], 3),
                "copy_same_bytes_us": round(fl["copy_3670016B_us"], 3),
                "kernel_us": round(kus, 3),
                "kernel_excess_over_empty_us": round(kus - fl["empty_kernel_us"], 3),
                "kernel_excess_over_copy_us": round(kus - fl["copy_3670016B_us"], 3),
                "hbm_time_at_peak_us": round(h["bytes"] / HBM_PEAK_GBS / 1e3, 3),
            }
    if not args.only_headline:
        try:
            line["configs"] = extra_configs(b, args)
        except Exception as e:  # report, never hide, a failing extra config
            line["configs_error"] = repr(e)
    if not args.only_headline:
        try:
            line["measured_ceilings"] = ceilings(b)
        except Exception as e:  # report, never hide
            line["measured_ceilings_error"] = repr(e)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_headline(args)
        if not args.only_headline:
            try:
                line["cpu_configs"] = cpu_configs(args)
            except Exception as e:  # report, never hide
                line["cpu_configs_error"] = repr(e)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
