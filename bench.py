"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--all] [--no-cpu]

Headline (the JSON line's `value`): the 4-bit decode GEMV at M=1, K=2048,
N=8192, group 64, bf16 out, as HBM GB/s of algorithmic bytes
(q + scales + biases + x + y = 9,457,664 B per launch). A step is one GEMV
launch over one weight copy; launches rotate over enough distinct copies
(>= 1 GiB) that the 256 MB Infinity Cache cannot hold them, so every step
streams its weights from HBM. The K timed steps run as one HIP graph replay
(back-to-back launches, no host in the loop), bracketed by synchronize and
hipEvents on the launch stream.

`roofline` reports the same kernel's average launch duration over that
replay (steps / event time), against the 8 TB/s HBM peak. The `gemm` object reports the
bf16 prefill GEMM at M=1024, K=2048, N=8192 (34.36 GFLOP) against the dense
bf16 MFMA peak. `cpu_baseline` times the CPU oracle (the reference's per-
element dequant check loop, restated in C) on the same workload on the host.
`--all` adds a per-config table (configs 0-4) to the JSON under "configs".
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 1 << 30


def measured_traffic():
    """HBM bytes per launch of the headline GEMV, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (scaled by a 256 MiB copy), or None."""
    import re

    path = os.path.join(ROOT, "profiles", "gemv4_k2048_n8192_hbm_traffic.md")
    try:
        m = re.search(r"gemv4_k2048_n8192_traffic_bytes=(\d+)", open(path).read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--all", action="store_true", help="also time every benchmark config")
    p.add_argument("--config", type=int, default=None, choices=range(5),
                   help="also time the cases of one benchmark config (0-4)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--calib-copy", action="store_true",
                   help="also run a 256 MiB device copy (reference for the HBM byte counters)")
    return p.parse_args()


class Timer:
    """Times a launch function over rotating operand sets.

    The timed steps are captured once into a HIP graph and replayed, so the
    launches run back to back with no host in the loop; the time is taken
    with hipEvents recorded on the launch stream around the replay, after a
    device synchronize. steps/time is the per-launch average duration (it
    agrees with rocprofv3's per-kernel average; see profiles/)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, steps, warmup):
        """Return (total_ms for `steps` launches, mode)."""
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        s0 = torch.cuda.Event(enable_timing=True)
        s1 = torch.cuda.Event(enable_timing=True)
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(steps):
                    fn(i)
            g.replay()  # the first replay uploads the graph
            torch.cuda.synchronize()
            s0.record()
            g.replay()
            s1.record()
            torch.cuda.synchronize()
            return s0.elapsed_time(s1), "hip-graph"
        except RuntimeError as e:
            print(f"[bench] graph capture failed ({e}); timing eager launches", file=sys.stderr)
        torch.cuda.synchronize()
        s0.record()
        for i in range(steps):
            fn(i)
        s1.record()
        torch.cuda.synchronize()
        return s0.elapsed_time(s1), "eager"


def gemv_case(torch, ops, synth, dev, bits, M, N, K, G, out_dtype, timer, steps, warmup):
    w = synth.quant_weights(N, K, G, bits, seed=synth.BASE_SEED + bits * 100 + M)
    base = ops.QuantLinear(w, dev)
    wbytes = w.nbytes
    copies = max(1, math.ceil(ROTATE_BYTES / wbytes))
    qs = [base.q] + [base.q.clone() for _ in range(copies - 1)]
    ss = [base.s] + [base.s.clone() for _ in range(copies - 1)]
    bs = [base.b] + [base.b.clone() for _ in range(copies - 1)]
    x = ops.to_device_bits(synth.activations(M, K), dev)
    y = torch.empty((M, N), dtype=out_dtype, device=dev)
    if bits == 4:
        f1, fb = ops.gemv4, ops.gemv4_b
    else:
        f1, fb = ops.gemv8, ops.gemv8_b

    def fn(i):
        j = i % copies
        if M == 1:
            f1(qs[j], ss[j], bs[j], x, y, N, K, group=G)
        else:
            fb(qs[j], ss[j], bs[j], x, y, N, K, M, group=G)

    # The same launches on one weight copy, served from the 256 MB Infinity
    # Cache once warm: reported under its own label, never as the headline.
    # Timed first, so the rotating (HBM) launches are the last in a trace.
    hot = None
    if copies > 1 and wbytes < 128 * 1024 * 1024:
        hot, _ = timer.run(lambda i: fn(0), steps, warmup)
    total, mode = timer.run(fn, steps, warmup)
    per = total / steps
    ybytes = M * N * (2 if out_dtype == torch.bfloat16 else 4)
    algo = wbytes + M * K * 2 + ybytes
    flops = 2.0 * M * N * K
    res = dict(M=M, N=N, K=K, G=G, bits=bits, bytes=algo, copies=copies, mode=mode,
               us_per_step=total * 1e3 / steps, us_kernel=per * 1e3,
               gbs_step=algo * steps / (total * 1e-3) / 1e9,
               gbs_kernel=algo / (per * 1e-3) / 1e9,
               tflops_kernel=flops / (per * 1e-3) / 1e12)
    res["hbm_frac_kernel"] = res["gbs_kernel"] / HBM_PEAK_GBS
    if hot is not None:
        res["us_hot_cache"] = hot * 1e3 / steps
        res["gbs_hot_cache"] = algo / (hot / steps * 1e-3) / 1e9
    del qs, ss, bs, base
    torch.cuda.empty_cache()
    return res


def gemm_case(torch, ops, synth, oracle_mod, dev, M, N, K, fused, timer, steps, warmup, G=64,
              vendor=False):
    w = synth.quant_weights(N, K, G, 4, seed=synth.BASE_SEED + N + K)
    lin = ops.QuantLinear(w, dev)
    A = ops.to_device_bits(synth.activations(M, K), dev)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if fused:
        wbytes = w.nbytes
        copies = max(1, math.ceil(ROTATE_BYTES / wbytes))
        qs = [lin.q] + [lin.q.clone() for _ in range(copies - 1)]
        ss = [lin.s] + [lin.s.clone() for _ in range(copies - 1)]
        bs = [lin.b] + [lin.b.clone() for _ in range(copies - 1)]

        def fn(i):
            j = i % copies
            ops.gemm_q4(A, qs[j], ss[j], bs[j], C, M, N, K, group=G)
    else:
        Bd = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
        ops.dequant_tile(lin.q, lin.s, lin.b, Bd, N, K, group=G)
        wbytes = N * K * 2
        copies = max(1, math.ceil(ROTATE_BYTES / wbytes))
        Bs = [Bd] + [Bd.clone() for _ in range(copies - 1)]

        def fn(i):
            ops.gemm_mpp(A, Bs[i % copies], C, M, N, K)

    total, mode = timer.run(fn, steps, warmup)
    per = total / steps
    flops = 2.0 * M * N * K
    algo = wbytes + M * K * 2 + M * N * 2
    vendor_us = None
    if vendor and not fused:
        # the vendor GEMM (torch.matmul -> hipBLASLt) on the same operands and rotation
        vt, _ = timer.run(lambda i: torch.matmul(A, Bs[i % copies].t(), out=C), steps, warmup)
        vendor_us = vt * 1e3 / steps
    res = dict(M=M, N=N, K=K, fused=fused, copies=copies, mode=mode,
               us_per_step=total * 1e3 / steps, us_kernel=per * 1e3,
               tflops_kernel=flops / (per * 1e-3) / 1e12,
               tflops_step=flops * steps / (total * 1e-3) / 1e12,
               gbs_kernel=algo / (per * 1e-3) / 1e9)
    res["mfma_frac_kernel"] = res["tflops_kernel"] / BF16_PEAK_TFLOPS
    if vendor_us is not None:
        res["vendor_us"] = vendor_us
        res["vendor_tflops"] = flops / (vendor_us * 1e-6) / 1e12
    res["hbm_frac_kernel"] = res["gbs_kernel"] / HBM_PEAK_GBS
    torch.cuda.empty_cache()
    return res


# One LFM-style layer's projections (name, K, N), BASELINE config 4.
LAYER = [("q", 2048, 2048), ("k", 2048, 512), ("v", 2048, 512), ("o", 2048, 2048),
         ("gate", 2048, 8192), ("up", 2048, 8192), ("down", 8192, 2048)]


class _Stacked:
    """Row-stacked weights of projections that read the same activation
    (q|k|v, gate|up): one product of N = sum of the parts, the same values
    per output row as the separate products."""

    def __init__(self, torch, lins):
        self.q = torch.cat([l.q for l in lins], 0)
        self.s = torch.cat([l.s for l in lins], 0)
        self.b = torch.cat([l.b for l in lins], 0)


def chain_case(torch, ops, synth, dev, M, timer, layers=24, G=64, steps=3, warmup=1,
               stacked=False):
    """Config 4: the fused 4-bit GEMM over a synthetic 24-layer projection
    chain (7 projections per layer, distinct random weights per layer), M
    activation rows. One step = the whole chain: 168 GEMMs, or with
    `stacked` 96, q|k|v and gate|up each one product on row-stacked weights
    (they read the same activation), as an engine lays them out."""
    ws = []
    for l in range(layers):
        lins = []
        for i, (name, K, N) in enumerate(LAYER):
            w = synth.quant_weights(N, K, G, 4, seed=synth.BASE_SEED + 1000 * l + i)
            lins.append((ops.QuantLinear(w, dev), K, N))
        if stacked:
            ws.append((_Stacked(torch, [x[0] for x in lins[0:3]]), 2048, 3072))
            ws.append(lins[3])
            ws.append((_Stacked(torch, [x[0] for x in lins[4:6]]), 2048, 16384))
            ws.append(lins[6])
            del lins
        else:
            ws.extend(lins)
    a2 = ops.to_device_bits(synth.activations(M, 2048), dev)
    a8 = ops.to_device_bits(synth.activations(M, 8192), dev)
    outs = {N: torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            for N in (512, 2048, 3072, 8192, 16384)}

    def fn(i):
        for lin, K, N in ws:
            ops.gemm_q4(a8 if K == 8192 else a2, lin.q, lin.s, lin.b, outs[N], M, N, K, group=G)

    total, mode = timer.run(fn, steps, warmup)
    per = total / steps
    flops = sum(2.0 * M * N * K for _, K, N in ws)
    wbytes = sum(l.q.numel() * 4 + l.s.numel() * 2 + l.b.numel() * 2 for l, _, _ in ws)
    res = dict(config=4, M=M, layers=layers, gemms=len(ws), stacked=stacked, mode=mode,
               us_per_chain=per * 1e3,
               tflops=flops / (per * 1e-3) / 1e12, weight_gbs=wbytes / (per * 1e-3) / 1e9,
               weight_bytes=wbytes, flops=flops)
    res["mfma_frac"] = res["tflops"] / BF16_PEAK_TFLOPS
    res["hbm_frac"] = res["weight_gbs"] / HBM_PEAK_GBS
    del ws
    torch.cuda.empty_cache()
    return res


def fused_decode_case(torch, ops, synth, dev, N, K, timer, steps, warmup, G=64):
    """Fused decode steps (rmsnorm -> gemv4 and silu_mul -> gemv4, as the
    reference's engine.cpp:388-400 runs them in two launches) against the
    plain gemv4 on the same rotating weights: the fused launch reads the fp32
    input (and the bf16 norm weight) instead of a bf16 activation."""
    w = synth.quant_weights(N, K, G, 4, seed=synth.BASE_SEED + 7 * N + K)
    base = ops.QuantLinear(w, dev)
    copies = max(1, math.ceil(ROTATE_BYTES / w.nbytes))
    qs = [base.q] + [base.q.clone() for _ in range(copies - 1)]
    ss = [base.s] + [base.s.clone() for _ in range(copies - 1)]
    bs = [base.b] + [base.b.clone() for _ in range(copies - 1)]
    xb = ops.to_device_bits(synth.activations(1, K), dev)
    xf = torch.randn(K, device=dev)
    up = torch.randn(K, device=dev)
    nw = (torch.rand(K, device=dev) + 0.5).to(torch.bfloat16)
    y = torch.empty(N, dtype=torch.bfloat16, device=dev)
    res = dict(N=N, K=K, G=G, copies=copies)
    cases = {
        "gemv4": (lambda j: ops.gemv4(qs[j], ss[j], bs[j], xb, y, N, K, group=G), K * 2),
        "rmsnorm_gemv4": (lambda j: ops.rmsnorm_gemv4(xf, nw, qs[j], ss[j], bs[j], y, N, K,
                                                      group=G), K * 6),
        "silu_mul_gemv4": (lambda j: ops.silu_mul_gemv4(xf, up, qs[j], ss[j], bs[j], y, N, K,
                                                        group=G), K * 8),
    }
    for name, (f, xbytes) in cases.items():
        total, mode = timer.run(lambda i: f(i % copies), steps, warmup)
        per = total / steps
        res[name + "_us"] = per * 1e3
        res[name + "_gbs"] = (w.nbytes + xbytes + N * 2) / (per * 1e-3) / 1e9
    res["mode"] = mode
    del qs, ss, bs, base
    torch.cuda.empty_cache()
    return res


def naive_case(torch, ops, dev, M, N, K, timer, steps, warmup):
    """gemm_naive, the any-shape fallback: C fp32 [M][N] = A [M][K] . B [N][K]^T,
    bf16 operands (the N=16 gate_proj and the bf16 batch lm_head)."""
    A = torch.randn(M, K, device=dev).to(torch.bfloat16)
    B = torch.randn(N, K, device=dev).to(torch.bfloat16)
    C = torch.empty(M, N, dtype=torch.float32, device=dev)
    total, mode = timer.run(lambda i: ops.gemm_naive(A, B, C, M, N, K, K, K, N), steps, warmup)
    per = total / steps
    algo = (M * K + N * K) * 2 + M * N * 4
    return dict(M=M, N=N, K=K, mode=mode, us_kernel=per * 1e3,
                gbs_kernel=algo / (per * 1e-3) / 1e9,
                tflops_kernel=2.0 * M * N * K / (per * 1e-3) / 1e12)


def calib_copy(torch, dev):
    """A plain 256 MiB device copy: reads and writes exactly 256 MiB, the
    reference for scaling FETCH_SIZE / WRITE_SIZE counters to bytes."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def launch_floors(torch, dev, timer, nbytes, steps):
    """What one launch of this size costs in vendor kernels on the same box,
    timed like the GEMV (HIP-graph replay, operands rotating over >= 1 GiB):
    an empty launch (a 1-element fill), and torch's device copy moving the
    same number of bytes (half read, half written)."""
    tiny = torch.empty(1, device=dev)
    t_fill, _ = timer.run(lambda i: tiny.zero_(), steps, 10)
    half = nbytes // 2 // 4
    copies = math.ceil(ROTATE_BYTES / (half * 4))
    srcs = [torch.empty(half, dtype=torch.int32, device=dev) for _ in range(copies)]
    dst = torch.empty(half, dtype=torch.int32, device=dev)
    t_copy, _ = timer.run(lambda i: dst.copy_(srcs[i % copies]), steps, 10)
    del srcs
    torch.cuda.empty_cache()
    return {"empty_launch_us": round(t_fill * 1e3 / steps, 3),
            "torch_copy_same_bytes_us": round(t_copy * 1e3 / steps, 3),
            "note": "vendor-kernel floors for one launch moving the GEMV's bytes"}


def cpu_baseline(seconds):
    """The oracle's faithful per-element GEMV (src/main.cpp:73-84 restated)
    on the headline workload, single-threaded, repeated for ~`seconds`."""
    import oracle
    from miori_amd import synth

    N, K, G = 8192, 2048, 64
    w = synth.quant_weights(N, K, G, 4, seed=synth.BASE_SEED + 400 + 1)
    x = synth.activations(1, K)
    algo = w.nbytes + K * 2 + N * 2
    oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, G, nthreads=1)  # warm
    t0 = time.perf_counter()
    reps = 0
    while True:
        oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, G, nthreads=1)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / reps
    nt = min(16, os.cpu_count() or 1)
    t1 = time.perf_counter()
    oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, G, nthreads=nt)
    per_mt = time.perf_counter() - t1
    return {"value": algo / per / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{reps} full passes of the 8192x2048 g64 4-bit GEMV (M=1), "
                      f"per-element dequant + fp64 accumulate, {per * 1e3:.1f} ms/pass",
            "threaded": {"value": algo / per_mt / 1e9, "cores": nt,
                         "sample": f"1 pass with OpenMP over {nt} threads, {per_mt * 1e3:.1f} ms"}}


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    import torch

    import oracle
    from miori_amd import _lib, ops, synth

    _lib.load()
    dev = torch.device("cuda:0")
    timer = Timer(torch)
    steps, warmup = args.steps, args.warmup

    head = gemv_case(torch, ops, synth, dev, 4, 1, 8192, 2048, 64, torch.bfloat16,
                     timer, steps, warmup)
    gemm = gemm_case(torch, ops, synth, oracle, dev, 1024, 8192, 2048, False, timer,
                     min(steps, 100), min(warmup, 10), vendor=True)
    floors = launch_floors(torch, dev, timer, head["bytes"], steps)

    out = {
        "metric": "4-bit GEMV HBM GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOP/s at M=1024",
        "value": round(head["gbs_step"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": head["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded splitmix64; MLX-affine 4-bit, group 64)",
        "config": {"workload": "gemv4 M=1 K=2048 N=8192 group=64 bf16-out, "
                               f"rotating {head['copies']} weight copies (HBM, not cache)",
                   "M": 1, "N": 8192, "K": 2048, "group": 64, "timing": head["mode"]},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs_kernel"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs_kernel"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(), "kernel_us": round(head["us_kernel"], 3),
                     "algorithmic_bytes": head["bytes"]},
        "gemm": {"workload": "bf16 GEMM M=1024 K=2048 N=8192, bf16 out",
                 "tflops": round(gemm["tflops_kernel"], 1),
                 "us": round(gemm["us_kernel"], 2),
                 "frac_of_bf16_peak": round(gemm["mfma_frac_kernel"], 4),
                 "hipblaslt_us_same_operands": round(gemm["vendor_us"], 2),
                 "hipblaslt_tflops": round(gemm["vendor_tflops"], 1)},
        "gemv_floors": floors,
        "gemv_hot_cache": {"us": round(head["us_hot_cache"], 3),
                           "gbs": round(head["gbs_hot_cache"], 1),
                           "note": "same launches on one weight copy (Infinity Cache "
                                   "resident); not the headline value"},
    }
    if args.calib_copy:
        calib_copy(torch, dev)
    if args.all or args.config is not None:
        out["configs"] = run_all(torch, ops, synth, oracle, dev, timer,
                                 only=None if args.all else args.config)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


def run_all(torch, ops, synth, oracle, dev, timer, only=None):
    """Every benchmark config, or only config `only` (0-4; the next-row cases,
    fused decode and gemm_naive, run with the full set)."""
    rows = []
    st, wu = 100, 10

    def want(c):
        return only is None or only == c

    def emit(row):
        rows.append(row)
        print(f"[bench] {row}", file=sys.stderr, flush=True)

    if want(0):
        emit(dict(config=0, **gemv_case(torch, ops, synth, dev, 4, 1, 8192, 2048, 64,
                                        torch.bfloat16, timer, st, wu)))
    if want(1):
        for (K, N) in [(2048, 2048), (2048, 512), (2048, 8192), (8192, 2048)]:
            for M in (2, 4, 8, 16, 32):
                emit(dict(config=1, **gemv_case(torch, ops, synth, dev, 4, M, N, K, 64,
                                                torch.bfloat16, timer, st, wu)))
    if want(2):
        for M in (1, 8, 32):
            emit(dict(config=2, **gemv_case(torch, ops, synth, dev, 8, M, 131072, 2048, 64,
                                            torch.bfloat16, timer, 20, 3)))
    if want(4):
        for M in (1024, 32):
            for stacked in (False, True):
                emit(chain_case(torch, ops, synth, dev, M, timer, stacked=stacked))
    for fused in (False, True):
        if not want(4 if fused else 3):
            continue
        for M in (256, 1024, 1472):
            for (K, N) in [(2048, 8192), (8192, 2048), (2048, 2560)]:
                emit(dict(config=4 if fused else 3,
                          **gemm_case(torch, ops, synth, oracle, dev, M, N, K, fused,
                                      timer, 30, 3)))
    if only is None:
        for (K, N) in [(2048, 2048), (2048, 8192), (7680, 2048), (8192, 2048)]:
            emit(dict(row="fused-decode", **fused_decode_case(torch, ops, synth, dev, N, K,
                                                             timer, st, wu)))
        for (M, N, K) in [(1, 16, 2048), (32, 16, 2048), (8, 131072, 2048), (32, 131072, 2048)]:
            emit(dict(row="gemm_naive", **naive_case(torch, ops, dev, M, N, K, timer, 20, 3)))
    return rows


if __name__ == "__main__":
    main()
