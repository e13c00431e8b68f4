"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]

Headline (the JSON line's `value`): the 4-bit decode GEMV at M=1, K=2048,
N=8192, group 64, bf16 out, as HBM GB/s of algorithmic bytes
(q + scales + biases + x + y = 9,457,664 B per launch). A step is one GEMV
launch over one weight copy.

Timing protocol (every row):
  * launches rotate over distinct operand copies totalling >= 1 GiB;
  * the K timed launches are captured once into a HIP graph; the graph is
    replayed once untimed (upload), then a 1 GiB buffer is read and written
    (evicting the 256 MB Infinity Cache and the L2s), then the timed replay
    runs, bracketed by synchronize and hipEvents on the launch stream. Every
    weight byte of the timed replay therefore comes from HBM, whatever K is;
    `copies_touched` and `bytes_touched` say how much distinct weight data
    the timed replay read;
  * the per-launch time is the replay time / K: back-to-back launches, so it
    includes the gap between kernels (the kernel trace in profiles/ gives
    the kernels' own durations).

The JSON line carries one row per BASELINE config (`configs`), each with
its roofline fraction, its floor on this box (`floor_us`: an empty launch
plus its algorithmic bytes at the vendor copy's streaming rate, and
`floor_frac` = floor / time, which is what a launch-bound small shape should
be judged by) and a CPU baseline: the CPU oracle (the reference's
per-element check loops, restated in C) timed single-threaded on a bounded
sample of the same workload on this host, extrapolated where stated. The
batch dispatch policy table (exact 4-bit batched GEMV vs the bf16-cache GEMM
vs the fused 4-bit GEMM, M = 1..32, config-1 shapes) is under `policy`.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 1 << 30
FLUSH_BYTES = 1 << 30


def measured_traffic():
    """HBM bytes per launch of the headline GEMV from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (scaled by a 256 MiB copy), or None."""
    import re

    path = os.path.join(ROOT, "profiles", "gemv4_k2048_n8192_hbm_traffic.md")
    try:
        m = re.search(r"gemv4_k2048_n8192_traffic_bytes=(\d+)", open(path).read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--quick", action="store_true",
                   help="headline, GEMM and config rows only (no policy table, no chain)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--headline-only", action="store_true",
                   help="only the config-0 GEMV and the launch floors (for counter passes)")
    p.add_argument("--case", default=None,
                   help="time one case only, KIND,M,N,K with KIND gemv4 | gemv8 | gemv4b | gemv8b "
                        "(batched entry at any M) | gemm_bf16 | gemm_q4 (for profiling runs)")
    p.add_argument("--clock", action="store_true",
                   help="also sample the shader clock during a GEMM replay (a side-stream "
                        "kernel; off by default)")
    p.add_argument("--diag-gemv", action="store_true",
                   help="per-wave wall-clock timeline of one cold headline GEMV launch "
                        "(miori_diag_gemv_q4_timeline), printed as one JSON line")
    p.add_argument("--calib-copy", action="store_true",
                   help="also run a 256 MiB device copy (reference for the HBM byte counters)")
    return p.parse_args()


def roofline(us, nbytes, flops):
    """Roofline of one launch: the bound is whichever of HBM (algorithmic
    bytes at 8 TB/s) and dense bf16 MFMA (flops at 2.5 PFLOP/s) takes longer."""
    t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
    t_mfma = flops / (BF16_PEAK_TFLOPS * 1e12)
    gbs = nbytes / (us * 1e-6) / 1e9
    tfs = flops / (us * 1e-6) / 1e12
    if t_hbm >= t_mfma:
        return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    return {"bound": "mfma", "achieved": round(tfs, 1), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tfs / BF16_PEAK_TFLOPS, 4)}


class Timer:
    """Times `steps` launches of fn(i) as one HIP-graph replay, with the
    caches flushed between the upload replay and the timed one."""

    def __init__(self, torch, dev):
        self.torch = torch
        self.flush = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)

    def _flush(self):
        self.flush.add_(1)  # reads and writes 1 GiB (about 0.3 ms)
        self.flush.add_(1)

    def run(self, fn, steps, warmup, pre=None):
        """Return (ms for `steps` launches, mode). `pre` (optional) is
        enqueued between the flush and the timed replay, e.g. to bring an
        operand back into the caches."""
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        s0 = torch.cuda.Event(enable_timing=True)
        s1 = torch.cuda.Event(enable_timing=True)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                fn(i)
        g.replay()  # the first replay uploads the graph
        torch.cuda.synchronize()
        # The flush is enqueued, not waited for: while the GPU works through
        # it, the host submits the timed replay, so the host-side graph
        # launch cost stays outside the events.
        self._flush()
        if pre is not None:
            pre()
        s0.record()
        g.replay()
        s1.record()
        torch.cuda.synchronize()
        del g
        return s0.elapsed_time(s1), "hip-graph, caches flushed (1 GiB) before the timed replay"


MFMA_PEAK_CLOCK_GHZ = 2.4  # the clock the dense bf16 peak is quoted at


def shader_clock(c, fn, steps):
    """Shader clock (GHz) while `steps` launches of fn(i) replay as a graph:
    miori_diag_clock_sample runs on a side stream beside the replay and
    records (s_memtime cycles, wall-clock ticks) pairs every 0.5 us; the clock
    of each interval is d(cycles) / d(ticks) x the wall-clock rate. The
    sampler holds one CU, so this replay is not the timed one."""
    import ctypes
    import numpy as np
    from miori_amd import _lib
    torch = c.torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    span_us = e0.elapsed_time(e1) * 1e3
    gap = 50  # ticks of the 100 MHz wall clock
    n = int(min(1 << 20, max(16, span_us * 100 / gap)))
    buf = torch.zeros(2 * n, dtype=torch.int64, device=c.dev)
    khz = ctypes.c_uint32(0)
    side = torch.cuda.Stream(device=c.dev)
    side.wait_stream(torch.cuda.current_stream())
    _lib.call("miori_diag_clock_sample", ctypes.c_void_p(buf.data_ptr()), n, gap,
              ctypes.byref(khz), ctypes.c_void_p(side.cuda_stream))
    g.replay()
    torch.cuda.synchronize()
    del g
    smp = buf.cpu().numpy().view(np.uint64).reshape(n, 2).astype(np.float64)
    # single 0.5 us intervals are quantised by the wall clock's resolution:
    # clocks are taken over 20-sample (10 us) windows and over the whole span
    w = 20
    dc = smp[w:, 0] - smp[:-w, 0]
    dr = smp[w:, 1] - smp[:-w, 1]
    ghz = dc[::w] / dr[::w] * khz.value * 1e3 / 1e9
    mean = (smp[-1, 0] - smp[0, 0]) / (smp[-1, 1] - smp[0, 1]) * khz.value * 1e3 / 1e9
    return {"mean_GHz": round(float(mean), 3), "median_GHz": round(float(np.median(ghz)), 3),
            "p10_GHz": round(float(np.percentile(ghz, 10)), 3),
            "p90_GHz": round(float(np.percentile(ghz, 90)), 3),
            "windows": int(ghz.size), "window_us": round(w * gap * 1e3 / khz.value, 1),
            "span_us": round(span_us, 1), "wall_clock_kHz": khz.value}


def _rotating(t, copies):
    return [t] + [t.clone() for _ in range(copies - 1)]


def _dev_quant(torch, dev, N, K, G, bits, gen):
    """Random MLX-affine weights made on the device (the benchmark
    distributions; a device generator, so large and many-layer cases need no
    host generation): q uniform words, scale ~ U(lo, hi), bias = -mid*scale
    (+ N(0, 1e-3) for 4-bit)."""
    words = N * K * bits // 32
    q = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, words // N), dtype=torch.int32, device=dev,
                      generator=gen)
    ng = K // G
    if bits == 4:
        s = (0.001 + 0.009 * torch.rand(N, ng, device=dev, generator=gen)).to(torch.bfloat16)
        b = (-8.0 * s.float() + 1e-3 * torch.randn(N, ng, device=dev, generator=gen)).to(torch.bfloat16)
    else:
        s = (1e-4 + 9e-4 * torch.rand(N, ng, device=dev, generator=gen)).to(torch.bfloat16)
        b = (-128.0 * s.float()).to(torch.bfloat16)
    return q, s, b


class Ctx:
    def __init__(self, torch, ops, synth, dev, timer, steps, warmup):
        self.torch, self.ops, self.synth, self.dev = torch, ops, synth, dev
        self.timer, self.steps, self.warmup = timer, steps, warmup
        self.gen = torch.Generator(device=dev)
        self.gen.manual_seed(0x4D494F52)


def gemv_row(c, bits, M, N, K, G=64, steps=None, hot=False, tag=None, batched=False):
    """Configs 0-2: the exact 4/8-bit GEMV (M = 1) or batched GEMV (M > 1, or
    any M with `batched`), bf16 out, on rotating weight copies."""
    torch, ops = c.torch, c.ops
    steps = steps or c.steps
    if bits == 8 and N >= 65536:
        q, s, b = _dev_quant(torch, c.dev, N, K, G, bits, c.gen)
    else:
        w = c.synth.quant_weights(N, K, G, bits, seed=c.synth.BASE_SEED + bits * 100 + M)
        lin = ops.QuantLinear(w, c.dev)
        q, s, b = lin.q, lin.s, lin.b
    wbytes = q.numel() * 4 + s.numel() * 2 + b.numel() * 2
    copies = max(1, math.ceil(ROTATE_BYTES / wbytes))
    qs, ss, bs = _rotating(q, copies), _rotating(s, copies), _rotating(b, copies)
    x = ops.to_device_bits(c.synth.activations(M, K), c.dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=c.dev)
    f1 = ops.gemv4 if bits == 4 else ops.gemv8
    fb = ops.gemv4_b if bits == 4 else ops.gemv8_b

    def fn(i):
        j = i % copies
        if M == 1 and not batched:
            f1(qs[j], ss[j], bs[j], x, y, N, K, group=G)
        else:
            fb(qs[j], ss[j], bs[j], x, y, N, K, M, group=G)

    total, mode = c.timer.run(fn, steps, c.warmup)
    us = total * 1e3 / steps
    nbytes = wbytes + M * K * 2 + M * N * 2
    flops = 2.0 * M * N * K
    row = dict(name=tag or f"gemv{bits}" + ("" if M == 1 else "_b"), M=M, N=N, K=K, G=G,
               us=round(us, 3), GB_s=round(nbytes / (us * 1e-6) / 1e9, 1),
               TFLOP_s=round(flops / (us * 1e-6) / 1e12, 2), bytes=nbytes, flops=flops,
               roofline=roofline(us, nbytes, flops), steps=steps, copies=copies,
               copies_touched=min(steps, copies), bytes_touched=steps * wbytes, timing=mode)
    if hot:
        th, _ = c.timer.run(lambda i: fn(0), steps, c.warmup)
        row["hot_cache_us"] = round(th * 1e3 / steps, 3)
    if M > 1:
        # x in the caches, weights still cold: a decode step finds x fresh
        # from the kernel that produced it, while the flush above evicts it
        # from L2 and the Infinity Cache like the weights
        xi = x.view(torch.int16)
        tx, _ = c.timer.run(fn, steps, 1, pre=lambda: xi.add_(0))
        row["x_hot_us"] = round(tx * 1e3 / steps, 3)
    del qs, ss, bs
    torch.cuda.empty_cache()
    return row


def gemm_row(c, M, N, K, fused, steps=30, vendor=False, G=64, clock=False):
    """Config 3 (bf16 weight cache) or config 4 (fused 4-bit), bf16 out."""
    torch, ops = c.torch, c.ops
    q, s, b = _dev_quant(torch, c.dev, N, K, G, 4, c.gen)
    A = ops.to_device_bits(c.synth.activations(M, K), c.dev)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=c.dev)
    if fused:
        wbytes = q.numel() * 4 + s.numel() * 2 + b.numel() * 2
        copies = max(1, math.ceil(ROTATE_BYTES / wbytes))
        qs, ss, bs = _rotating(q, copies), _rotating(s, copies), _rotating(b, copies)

        def fn(i):
            j = i % copies
            ops.gemm_q4(A, qs[j], ss[j], bs[j], C, M, N, K, group=G)
    else:
        Bd = torch.empty((N, K), dtype=torch.bfloat16, device=c.dev)
        ops.dequant_tile(q, s, b, Bd, N, K, group=G)
        wbytes = N * K * 2
        copies = max(1, math.ceil(ROTATE_BYTES / wbytes))
        Bs = _rotating(Bd, copies)

        def fn(i):
            ops.gemm_mpp(A, Bs[i % copies], C, M, N, K)

    total, mode = c.timer.run(fn, steps, min(c.warmup, 5))
    us = total * 1e3 / steps
    flops = 2.0 * M * N * K
    nbytes = wbytes + M * K * 2 + M * N * 2
    row = dict(name="gemm_q4_fused" if fused else "gemm_bf16", M=M, N=N, K=K,
               us=round(us, 2), TFLOP_s=round(flops / (us * 1e-6) / 1e12, 1),
               GB_s=round(nbytes / (us * 1e-6) / 1e9, 1), flops=flops, bytes=nbytes,
               roofline=roofline(us, nbytes, flops), steps=steps, copies=copies,
               copies_touched=min(steps, copies), bytes_touched=steps * wbytes, timing=mode)
    if clock:
        clk = shader_clock(c, fn, steps)
        clk["mfma_peak_at_clock_TFLOP_s"] = round(
            BF16_PEAK_TFLOPS * clk["mean_GHz"] / MFMA_PEAK_CLOCK_GHZ, 1)
        clk["frac_at_clock"] = round(row["TFLOP_s"] / clk["mfma_peak_at_clock_TFLOP_s"], 4)
        row["clock"] = clk
    if vendor and not fused:
        vfn = lambda i: torch.matmul(A, Bs[i % copies].t(), out=C)  # noqa: E731
        vt, _ = c.timer.run(vfn, steps, 5)
        row["hipblaslt_us"] = round(vt * 1e3 / steps, 2)
        row["hipblaslt_TFLOP_s"] = round(flops / (vt * 1e-3 / steps) / 1e12, 1)
        if clock:
            row["hipblaslt_clock"] = shader_clock(c, vfn, steps)
    torch.cuda.empty_cache()
    return row


# One LFM-style layer's projections (name, K, N), BASELINE config 4.
LAYER = [("q", 2048, 2048), ("k", 2048, 512), ("v", 2048, 512), ("o", 2048, 2048),
         ("gate", 2048, 8192), ("up", 2048, 8192), ("down", 8192, 2048)]


def chain_row(c, M, stacked, layers=24, G=64, steps=3):
    """Config 4: the fused 4-bit GEMM over a synthetic 24-layer projection
    chain (7 projections per layer, distinct random weights per layer). One
    step = the whole chain: 168 GEMMs, or with `stacked` 96, where q|k|v and
    gate|up (which read the same activation) are each one product over
    row-stacked weights. The 821 MB of weights exceed the Infinity Cache."""
    torch, ops = c.torch, c.ops
    ws = []
    for _ in range(layers):
        parts = [(_dev_quant(torch, c.dev, N, K, G, 4, c.gen), K, N) for _, K, N in LAYER]
        if stacked:
            def cat(ps):
                return tuple(torch.cat([p[0][i] for p in ps], 0) for i in range(3))
            ws += [(cat(parts[0:3]), 2048, 3072), parts[3], (cat(parts[4:6]), 2048, 16384),
                   parts[6]]
        else:
            ws += parts
    a2 = ops.to_device_bits(c.synth.activations(M, 2048), c.dev)
    a8 = ops.to_device_bits(c.synth.activations(M, 8192), c.dev)
    outs = {N: torch.empty((M, N), dtype=torch.bfloat16, device=c.dev)
            for N in (512, 2048, 3072, 8192, 16384)}

    def fn(i):
        for (q, s, b), K, N in ws:
            ops.gemm_q4(a8 if K == 8192 else a2, q, s, b, outs[N], M, N, K, group=G)

    total, mode = c.timer.run(fn, steps, 1)
    us = total * 1e3 / steps
    flops = sum(2.0 * M * N * K for _, K, N in ws)
    wbytes = sum(q.numel() * 4 + s.numel() * 2 + b.numel() * 2 for (q, s, b), _, _ in ws)
    nbytes = wbytes + sum(M * K * 2 + M * N * 2 for _, K, N in ws)
    row = dict(name="chain_q4_fused" + ("_stacked" if stacked else ""), M=M, layers=layers,
               gemms=len(ws), us=round(us, 1), TFLOP_s=round(flops / (us * 1e-6) / 1e12, 1),
               weight_GB_s=round(wbytes / (us * 1e-6) / 1e9, 1), flops=flops, bytes=nbytes,
               roofline=roofline(us, nbytes, flops), steps=steps, bytes_touched=steps * wbytes,
               timing=mode)
    del ws
    torch.cuda.empty_cache()
    return row


def policy_table(c, steps=50):
    """Batch dispatch policy (BatchEngine::linear, src/batch.cpp:223-230):
    per config-1 shape and M = 1..32, µs of the exact 4-bit batched GEMV
    (what miori_linear_q4 runs), of the bf16-cache GEMM the reference runs
    above 4 slots, and of the fused 4-bit GEMM, all on rotating weights."""
    torch, ops = c.torch, c.ops
    out = []
    for K, N in [(2048, 2048), (2048, 512), (2048, 8192), (8192, 2048)]:
        q, s, b = _dev_quant(torch, c.dev, N, K, 64, 4, c.gen)
        w4 = q.numel() * 4 + s.numel() * 2 + b.numel() * 2
        c4 = max(1, math.ceil(ROTATE_BYTES / w4))
        qs, ss, bs = _rotating(q, c4), _rotating(s, c4), _rotating(b, c4)
        Bd = torch.empty((N, K), dtype=torch.bfloat16, device=c.dev)
        ops.dequant_tile(q, s, b, Bd, N, K)
        cb = max(1, math.ceil(ROTATE_BYTES / (N * K * 2)))
        Bs = _rotating(Bd, cb)
        x = ops.to_device_bits(c.synth.activations(32, K), c.dev)
        y = torch.empty((32, N), dtype=torch.bfloat16, device=c.dev)
        rec = {"K": K, "N": N, "M": [], "exact_us": [], "bf16_cache_us": [], "fused_us": []}
        for M in range(1, 33):
            xm, ym = x[:M], y[:M]
            te, _ = c.timer.run(lambda i: ops.linear(xm, qs[i % c4], ss[i % c4], bs[i % c4], ym,
                                                     M, N, K), steps, 3)
            tc, _ = c.timer.run(lambda i: ops.gemm_mpp(xm, Bs[i % cb], ym, M, N, K), steps, 3)
            tf, _ = c.timer.run(lambda i: ops.gemm_q4(xm, qs[i % c4], ss[i % c4], bs[i % c4], ym,
                                                      M, N, K), steps, 3)
            rec["M"].append(M)
            rec["exact_us"].append(round(te * 1e3 / steps, 2))
            rec["bf16_cache_us"].append(round(tc * 1e3 / steps, 2))
            rec["fused_us"].append(round(tf * 1e3 / steps, 2))
        rec["exact_beats_bf16_cache_at_every_M"] = all(
            e < cc for e, cc in zip(rec["exact_us"], rec["bf16_cache_us"]))
        out.append(rec)
        print(f"[bench] policy {rec}", file=sys.stderr, flush=True)
        del qs, ss, bs, Bs
        torch.cuda.empty_cache()
    return out


def fused_decode_row(c, N, K, steps=100, G=64):
    """Fused decode steps (rmsnorm -> gemv4 and silu_mul -> gemv4, which the
    reference's engine.cpp:388-400 runs as two launches) against the plain
    gemv4 on the same rotating weights."""
    torch, ops = c.torch, c.ops
    q, s, b = _dev_quant(torch, c.dev, N, K, G, 4, c.gen)
    wbytes = q.numel() * 4 + s.numel() * 2 + b.numel() * 2
    copies = max(1, math.ceil(ROTATE_BYTES / wbytes))
    qs, ss, bs = _rotating(q, copies), _rotating(s, copies), _rotating(b, copies)
    xb = ops.to_device_bits(c.synth.activations(1, K), c.dev)
    xf = torch.randn(K, device=c.dev)
    up = torch.randn(K, device=c.dev)
    nw = (torch.rand(K, device=c.dev) + 0.5).to(torch.bfloat16)
    y = torch.empty(N, dtype=torch.bfloat16, device=c.dev)
    row = dict(name="fused_decode", N=N, K=K, G=G)
    for name, f in {
        "gemv4": lambda j: ops.gemv4(qs[j], ss[j], bs[j], xb, y, N, K, group=G),
        "rmsnorm_gemv4": lambda j: ops.rmsnorm_gemv4(xf, nw, qs[j], ss[j], bs[j], y, N, K, group=G),
        "silu_mul_gemv4": lambda j: ops.silu_mul_gemv4(xf, up, qs[j], ss[j], bs[j], y, N, K,
                                                       group=G),
    }.items():
        t, _ = c.timer.run(lambda i: f(i % copies), steps, 5)
        row[name + "_us"] = round(t * 1e3 / steps, 3)
    del qs, ss, bs
    torch.cuda.empty_cache()
    return row


def naive_row(c, M, N, K, steps=20):
    """gemm_naive, the any-shape fallback (bf16 operands, fp32 C)."""
    torch, ops = c.torch, c.ops
    A = torch.randn(M, K, device=c.dev).to(torch.bfloat16)
    B = torch.randn(N, K, device=c.dev).to(torch.bfloat16)
    C = torch.empty(M, N, dtype=torch.float32, device=c.dev)
    t, _ = c.timer.run(lambda i: ops.gemm_naive(A, B, C, M, N, K, K, K, N), steps, 3)
    us = t * 1e3 / steps
    return dict(name="gemm_naive", M=M, N=N, K=K, us=round(us, 2),
                TFLOP_s=round(2.0 * M * N * K / (us * 1e-6) / 1e12, 1))


def launch_floors(c, nbytes, steps):
    """Vendor kernels timed like the GEMV on the same box: an empty launch
    (a 1-element fill) and torch's device copy moving the GEMV's bytes (half
    read, half written), sources rotating over >= 1 GiB."""
    torch = c.torch
    tiny = torch.empty(1, device=c.dev)
    t_fill, _ = c.timer.run(lambda i: tiny.zero_(), steps, 10)
    half = nbytes // 2 // 4
    copies = math.ceil(ROTATE_BYTES / (half * 4))
    srcs = [torch.empty(half, dtype=torch.int32, device=c.dev) for _ in range(copies)]
    dst = torch.empty(half, dtype=torch.int32, device=c.dev)
    t_copy, _ = c.timer.run(lambda i: dst.copy_(srcs[i % copies]), steps, 10)
    # streaming rate of the vendor copy on a large buffer (1 GiB read + 1 GiB
    # written per launch, so launch overhead is negligible): the rate the
    # per-row floors below use
    big = torch.empty(ROTATE_BYTES // 4, dtype=torch.int32, device=c.dev)
    big2 = torch.empty_like(big)
    t_big, _ = c.timer.run(lambda i: big2.copy_(big), 3, 1)
    del big, big2, srcs
    torch.cuda.empty_cache()
    return {"empty_launch_us": round(t_fill * 1e3 / steps, 3),
            "torch_copy_same_bytes_us": round(t_copy * 1e3 / steps, 3),
            "copy_stream_GB_s": round(2 * ROTATE_BYTES / (t_big * 1e-3 / 3) / 1e9, 1)}


def add_floor(row, floors):
    """Floor of one launch on this box: an empty launch plus the row's
    algorithmic bytes at the vendor copy's streaming rate. `floor_frac` =
    floor / measured time, so a small, launch-bound shape is not read as
    kernel inefficiency its roofline fraction cannot show."""
    fl = floors["empty_launch_us"] + row["bytes"] / (floors["copy_stream_GB_s"] * 1e3)
    row["floor_us"] = round(fl, 3)
    row["floor_frac"] = round(fl / row["us"], 4)
    return row


def gemv_timeline(c, N=8192, K=2048, G=64, reps=5):
    """Decompose cold headline GEMV launches with the stamped diagnostic
    build: per wave, the wall-clock time from the first wave's start to
    its own start, to its loads landing, to its arithmetic done and to its
    stores completing. Each launch follows a 1 GiB flush on a fresh weight
    copy. Percentiles over waves, median over launches."""
    import numpy as np
    torch, ops = c.torch, c.ops
    w = c.synth.quant_weights(N, K, G, 4, seed=c.synth.BASE_SEED + 900)
    lin = ops.QuantLinear(w, c.dev)
    x = ops.to_device_bits(c.synth.activations(1, K), c.dev)
    y = torch.empty(N, dtype=torch.bfloat16, device=c.dev)
    keys = ("start", "landed", "math_done", "stored")
    runs = []
    for r in range(reps):
        q, s, b = lin.q.clone(), lin.s.clone(), lin.b.clone()
        torch.cuda.synchronize()
        c.timer._flush()
        st = ops.gemv4_timeline(q, s, b, x, y, N, K, group=G)
        torch.cuda.synchronize()
        a = st.cpu().numpy().astype(np.int64)
        a = a - a[:, 0].min()
        runs.append({k: np.percentile(a[:, i], [0, 10, 50, 90, 100]) for i, k in enumerate(keys)})
        runs[-1]["compute"] = np.percentile(a[:, 2] - a[:, 1], [0, 10, 50, 90, 100])
        runs[-1]["after_last_landed"] = a[:, 3].max() - a[:, 1].max()
    # ticks per microsecond from the device's wall-clock rate
    import ctypes
    from miori_amd import _lib
    khz = ctypes.c_uint32(0)
    smp = torch.zeros(4, dtype=torch.int64, device=c.dev)
    _lib.call("miori_diag_clock_sample", ctypes.c_void_p(smp.data_ptr()), 2, 1,
              ctypes.byref(khz), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    tpu = khz.value / 1000.0
    out = {"unit": "us from the first wave's start", "wall_clock_kHz": khz.value,
           "percentiles": [0, 10, 50, 90, 100], "waves": int(a.shape[0]), "launches": reps}
    for k in keys + ("compute",):
        med = np.median(np.stack([r[k] for r in runs]), axis=0) / tpu
        out[k] = [round(float(v), 3) for v in med]
    out["last_landed_to_last_store_us"] = round(
        float(np.median([r["after_last_landed"] for r in runs])) / tpu, 3)
    return out


def calib_copy(torch, dev):
    """A plain 256 MiB device copy, three times: it reads and writes exactly
    256 MiB per launch, the reference for scaling FETCH_SIZE / WRITE_SIZE."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


# ---------------------------------------------------------------- CPU baselines
def _timed(fn, budget):
    """Run fn() at least once and until `budget` seconds; seconds per call."""
    fn()  # warm
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget:
            return el / n, n


def cpu_baselines(synth, budget=2.5):
    """The oracle on a bounded sample of each config's workload, scaled to
    the GPU row's unit: single-threaded (the reference's faithful check
    loop, `cores` = 1) and, under `threaded`, the same loop split over the
    host's cores with OpenMP. Returns {config: baseline}."""
    import numpy as np

    import oracle

    nt = min(16, os.cpu_count() or 1)
    out = {}

    def pair(fn, fn_mt, scale, unit, work, sample, b=budget):
        per, n = _timed(fn, b)
        per_mt, n_mt = _timed(fn_mt, b / 4)
        full, full_mt = per * scale, per_mt * scale
        return {"value": round(work / full, 6), "unit": unit, "cores": 1, "kind": "port",
                "us": round(full * 1e6, 1),
                "sample": sample.format(n=n, ms=per * 1e3),
                "threaded": {"value": round(work / full_mt, 6), "cores": nt,
                             "us": round(full_mt * 1e6, 1),
                             "sample": f"{n_mt} passes of the same sample, OpenMP over {nt} "
                                       f"threads, {per_mt * 1e3:.1f} ms each"}}

    # config 0: full 8192 x 2048 g64 4-bit GEMV, M = 1 (src/main.cpp:73-84)
    w = synth.quant_weights(8192, 2048, 64, 4, seed=synth.BASE_SEED + 401)
    x = synth.activations(1, 2048)
    out[0] = pair(lambda: oracle.gemv_f64(w.q, w.s, w.b, x, 4, 2048, 64, nthreads=1),
                  lambda: oracle.gemv_f64(w.q, w.s, w.b, x, 4, 2048, 64, nthreads=nt),
                  1, "GB/s", (w.nbytes + 4096 + 16384) / 1e9,
                  "{n} full passes of the 8192x2048 g64 4-bit GEMV (M=1), per-element dequant "
                  "+ fp64 accumulate, {ms:.1f} ms/pass", budget * 2)
    # config 1: gate/up 2048 -> 8192 at M = 8, rows [0, 1024) extrapolated to 8192
    x8 = synth.activations(8, 2048)
    out[1] = pair(lambda: oracle.gemv_rows_f64(w.q, w.s, w.b, x8, 4, 2048, 64, 0, 1024),
                  lambda: oracle.gemv_rows_f64(w.q, w.s, w.b, x8, 4, 2048, 64, 0, 1024,
                                               nthreads=nt),
                  8, "GB/s", (w.nbytes + 8 * 4096 + 8 * 8192 * 2) / 1e9,
                  "{n} passes over output rows 0..1023 of the 2048->8192 g64 GEMV at M=8, "
                  "{ms:.1f} ms each, x8 extrapolated to all 8192 rows")
    # config 2: 8-bit lm_head M = 1, a 2048-row slice extrapolated to 131072
    w8 = synth.quant_weights(2048, 2048, 64, 8, seed=synth.BASE_SEED + 402)
    out[2] = pair(lambda: oracle.gemv_f64(w8.q, w8.s, w8.b, x, 8, 2048, 64, nthreads=1),
                  lambda: oracle.gemv_f64(w8.q, w8.s, w8.b, x, 8, 2048, 64, nthreads=nt),
                  64, "GB/s", (131072 * (2048 + 2 * 32 * 2) + 4096 + 131072 * 2) / 1e9,
                  "{n} passes of a 2048-row slice of the 8-bit g64 lm_head (M=1), {ms:.1f} ms "
                  "each, x64 extrapolated to 131072 rows")
    # configs 3 / 4: M=1024, K=2048, N=8192; 16 rows of A, extrapolated to 1024
    A = synth.activations(16, 2048)
    Bq = synth.quant_weights(8192, 2048, 64, 4, seed=synth.BASE_SEED + 403)
    Bb = oracle.dequant_bf16(Bq.q, Bq.s, Bq.b, 4, 2048, 64)
    rows = np.arange(16, dtype=np.int64)
    tflop = 2.0 * 1024 * 8192 * 2048 / 1e12
    out[3] = pair(lambda: oracle.gemm_bf16_f64(A, Bb, rows, nthreads=1),
                  lambda: oracle.gemm_bf16_f64(A, Bb, rows, nthreads=nt),
                  64, "TFLOP/s", tflop,
                  "{n} passes of 16 rows x 8192 x 2048 (src/main.cpp:594-601 loop, fp64 "
                  "accumulate), {ms:.0f} ms each, x64 extrapolated to M=1024")
    per_d, nd = _timed(lambda: oracle.dequant_bf16(Bq.q, Bq.s, Bq.b, 4, 2048, 64), budget / 2)
    c3 = out[3]
    full4 = per_d + c3["us"] * 1e-6
    full4_mt = per_d + c3["threaded"]["us"] * 1e-6
    out[4] = {"value": round(tflop / full4, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
              "us": round(full4 * 1e6, 1),
              "sample": f"dequant of the 8192x2048 g64 weights ({per_d * 1e3:.0f} ms, {nd} "
                        "passes) + the config-3 GEMM sample, for one M=1024 projection",
              "threaded": {"value": round(tflop / full4_mt, 6), "cores": nt,
                           "us": round(full4_mt * 1e6, 1),
                           "sample": "the same dequant (single thread) + the threaded GEMM "
                                     "sample"}}
    return out


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    import torch

    from miori_amd import _lib, ops, synth

    _lib.load()
    dev = torch.device("cuda:0")
    c = Ctx(torch, ops, synth, dev, Timer(torch, dev), args.steps, args.warmup)
    t_start = time.time()

    def log(row):
        print(f"[bench] {row}", file=sys.stderr, flush=True)
        return row

    if args.diag_gemv:
        print(json.dumps({"gemv4_timeline": gemv_timeline(c)}), flush=True)
        return
    if args.case:
        kind, M, N, K = args.case.split(",")
        M, N, K = int(M), int(N), int(K)
        if kind in ("gemv4", "gemv8"):
            row = gemv_row(c, 4 if kind == "gemv4" else 8, M, N, K)
        elif kind in ("gemv4b", "gemv8b"):
            # the batched entry point at any M (with MIORI_BATCH_MFMA_MIN_M
            # this times the MFMA kernel at M < 5)
            row = gemv_row(c, 4 if kind == "gemv4b" else 8, M, N, K, batched=True)
        elif kind in ("gemm_bf16", "gemm_q4"):
            row = gemm_row(c, M, N, K, kind == "gemm_q4", steps=min(args.steps, 30),
                           vendor=args.clock and kind == "gemm_bf16", clock=args.clock)
        else:
            raise SystemExit(f"unknown case kind {kind}")
        if args.calib_copy:
            calib_copy(torch, dev)
        print(json.dumps(row), flush=True)
        return
    head = log(gemv_row(c, 4, 1, 8192, 2048, hot=True, tag="gemv4"))
    floors = launch_floors(c, head["bytes"], args.steps)
    if args.headline_only:
        if args.calib_copy:
            calib_copy(torch, dev)
        print(json.dumps({"gemv4": head, "gemv_floors": floors}), flush=True)
        return
    gemm = log(gemm_row(c, 1024, 8192, 2048, False, steps=min(args.steps, 100), vendor=True,
                        clock=args.clock))

    rows = [dict(config=0, **add_floor(dict(head), floors))]
    for K, N in [(2048, 8192), (2048, 2048), (2048, 512), (8192, 2048)]:
        for M in (2, 4, 8, 16, 32):
            rows.append(log(dict(config=1, **add_floor(gemv_row(c, 4, M, N, K, steps=100),
                                                        floors))))
    for M in (1, 8, 32):
        rows.append(log(dict(config=2, **add_floor(gemv_row(c, 8, M, 131072, 2048, steps=20,
                                                            tag="gemv8_lm_head"), floors))))
    for fused in (False, True):
        for M in (256, 1024, 1472):
            for K, N in [(2048, 8192), (8192, 2048), (2048, 2560)]:
                rows.append(log(dict(config=4 if fused else 3,
                                     **add_floor(gemm_row(c, M, N, K, fused, vendor=not fused),
                                                 floors))))
    extra = {}
    if not args.quick:
        for M in (1024, 32):
            for stacked in (False, True):
                rows.append(log(dict(config=4, **chain_row(c, M, stacked))))
        extra["policy"] = policy_table(c)
        nxt = []
        for K, N in [(2048, 2048), (2048, 8192), (8192, 2048)]:
            nxt.append(log(fused_decode_row(c, N, K)))
        for M, N, K in [(1, 16, 2048), (32, 16, 2048), (8, 131072, 2048), (32, 131072, 2048)]:
            nxt.append(log(naive_row(c, M, N, K)))
        extra["next_rows"] = nxt

    cpu = None if args.no_cpu else cpu_baselines(synth)
    if cpu:
        for r in rows:
            base = cpu.get(r["config"])
            if base is None:
                continue
            same = ((r["config"] == 0) or (r["config"] == 1 and r["M"] == 8 and r["N"] == 8192
                                           and r["K"] == 2048)
                    or (r["config"] == 2 and r["M"] == 1)
                    or (r["config"] in (3, 4) and r.get("name", "").startswith("gemm")
                        and (r["M"], r["N"], r["K"]) == (1024, 8192, 2048)))
            if same:
                r["cpu_baseline"] = base
    if args.calib_copy:
        calib_copy(torch, dev)

    wbytes_head = head["bytes"] - 2048 * 2 - 8192 * 2
    out = {
        "metric": "4-bit GEMV HBM GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOP/s at M=1024",
        "value": head["GB_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes, bf16 scale/bias/x, fp32 accumulate, bf16 out",
        "data": "synthetic (seeded splitmix64 / device RNG; MLX-affine, group 64)",
        "config": {"workload": "gemv4 M=1 K=2048 N=8192 group=64 bf16-out (BASELINE config 0)",
                   "M": 1, "N": 8192, "K": 2048, "group": 64, "timing": head["timing"],
                   "copies": head["copies"], "copies_touched": head["copies_touched"],
                   "bytes_touched": head["bytes_touched"], "flush_bytes": FLUSH_BYTES,
                   "weight_bytes_per_copy": wbytes_head},
        "roofline": {**head["roofline"], "traffic": measured_traffic(),
                     "traffic_source": "from profiles/gemv4_k2048_n8192_hbm_traffic.md, not "
                                       "this run (rocprofv3 FETCH_SIZE + WRITE_SIZE passes of "
                                       "the same kernel, scaled by a 256 MiB copy)",
                     "traffic_measured_in_this_run": False,
                     "launch_us": head["us"], "algorithmic_bytes": head["bytes"]},
        "gemm": {"workload": "bf16 GEMM M=1024 K=2048 N=8192, bf16 out (config 3)",
                 "us": gemm["us"], "TFLOP_s": gemm["TFLOP_s"], "roofline": gemm["roofline"],
                 "hipblaslt_us": gemm["hipblaslt_us"],
                 "hipblaslt_TFLOP_s": gemm["hipblaslt_TFLOP_s"],
                 "clock": gemm.get("clock"), "hipblaslt_clock": gemm.get("hipblaslt_clock")},
        "gemv_floors": floors,
        "gemv_hot_cache_us": head["hot_cache_us"],
        "configs": rows,
        **extra,
    }
    if cpu:
        out["cpu_baseline"] = cpu[0]
        out["cpu_model"] = cpu_model()
        out["cpu_threads_available"] = os.cpu_count()
    out["bench_wall_s"] = round(time.time() - t_start, 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
