"""Every BASELINE config sub-shape the benchmark times, checked against the
oracle at that exact shape (the benchmark's tolerance, tests/_check.py):

* config 1 (batched 4-bit GEMV, the fixed-slot batch decode of
  src/batch.cpp:223-230): gate/up 2048 -> 8192 and down 8192 -> 2048 at
  M = 2, 8, 16 (down at M = 16 takes the skinny kernel's 4-way K split),
  q/o 2048 -> 2048 and k/v 2048 -> 512 at M = 8 and 32;
* config 4 (fused dequant-in-LDS 4-bit GEMM): the stacked q|k|v (N = 3072)
  and gate|up (N = 16384) products at M = 32 and 1024, the fused
  M = 1024 down projection (K = 8192, N = 2048), and k/v (N = 512) at
  M = 32 and 1024;
* the batch dispatch entry (miori_linear_q4, BatchEngine::linear) at M = 8
  and M = 64 with and without a bf16 cache.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from miori_amd import ops, synth
from tests._check import check_close
from tests.gpu_util import acts, say, strided_rows, weights

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


@pytest.mark.parametrize("K,N,M", [
    (2048, 8192, 2), (2048, 8192, 8), (2048, 8192, 16),
    (8192, 2048, 2), (8192, 2048, 8), (8192, 2048, 16),
    (2048, 2048, 8), (2048, 2048, 32), (2048, 512, 8), (2048, 512, 32),
])
def test_config1_batched_gemv(dev, K, N, M):
    say(f"config1 gemv4_b K={K} N={N} M={M}")
    w, lin = weights(N, K, 64, 4, seed=1000 + N + K + M, dev=dev)
    x, xd = acts(M, K, seed=2000 + M, dev=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ops.gemv4_b(lin.q, lin.s, lin.b, xd, y, N, K, M)
    torch.cuda.synchronize()
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, 64, nthreads=NT)
    check_close(ops.bits_of(y), ref, f"config1 {K}->{N} M={M}")


@pytest.mark.parametrize("M,K,N", [
    (32, 2048, 3072), (1024, 2048, 3072), (32, 2048, 16384), (1024, 2048, 16384),
    (1024, 8192, 2048), (32, 2048, 512), (1024, 2048, 512),
])
def test_config4_fused_shapes(dev, M, K, N):
    say(f"config4 gemm_q4 M={M} K={K} N={N}")
    w = synth.quant_weights(N, K, 64, 4, seed=3000 + M + N + K)
    lin = ops.QuantLinear(w, dev)
    A = synth.activations(M, K, seed=4000 + M)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ops.gemm_q4(ops.to_device_bits(A, dev), lin.q, lin.s, lin.b, C, M, N, K)
    torch.cuda.synchronize()
    rows = np.arange(M, dtype=np.int64) if M <= 64 else strided_rows(M, 61)
    Bbits = oracle.dequant_bf16(w.q, w.s, w.b, 4, K, 64)
    ref = oracle.gemm_bf16_f64(A, Bbits, rows, nthreads=NT)
    check_close(ops.bits_of(C)[rows], ref, f"config4 {M}x{K}x{N}")


@pytest.mark.parametrize("M", [8, 64])
def test_linear_dispatch(dev, M):
    """miori_linear_q4: M <= 32 is the exact 4-bit batched GEMV (the fp64
    oracle of the fp32 dequant); M > 32 is the bf16-cache GEMM when a cache
    is given, else the fused GEMM, bit-identical to each other."""
    K, N = 2048, 2048
    say(f"linear M={M}")
    w, lin = weights(N, K, 64, 4, seed=5000 + M, dev=dev)
    x, xd = acts(M, K, seed=6000 + M, dev=dev)
    cache = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    ops.dequant_tile(lin.q, lin.s, lin.b, cache, N, K)
    y1 = torch.empty((M, N), dtype=torch.float32, device=dev)
    y2 = torch.empty_like(y1)
    ops.linear(xd, lin.q, lin.s, lin.b, y1, M, N, K, bf16_cache=cache)
    ops.linear(xd, lin.q, lin.s, lin.b, y2, M, N, K)
    torch.cuda.synchronize()
    if M <= 32:
        ref = oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, 64, nthreads=NT)
        ye = torch.empty_like(y1)
        ops.gemv4_b(lin.q, lin.s, lin.b, xd, ye, N, K, M)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ops.bits_of(y1), ops.bits_of(ye))
    else:
        Bbits = oracle.dequant_bf16(w.q, w.s, w.b, 4, K, 64)
        ref = oracle.gemm_bf16_f64(x, Bbits, np.arange(M, dtype=np.int64), nthreads=NT)
    check_close(ops.bits_of(y1), ref, f"linear M={M}")
    np.testing.assert_array_equal(ops.bits_of(y1), ops.bits_of(y2))
