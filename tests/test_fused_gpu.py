"""GPU parity of the fused decode ops: rmsnorm -> gemv4 and silu_mul -> gemv4
(the reference's separate kernels shaders/ops.metal:86-114, 129-139 and
6-42 as called in src/engine.cpp:388-400), against the oracle: the CPU
restatement of the transform (bf16 activation) followed by the fp64 GEMV,
under the benchmark tolerance. The transform's fp32 sums and rsqrt / exp may
round differently from the CPU in the last ulp, which moves a few bf16
activations by one ulp; the tolerance covers it."""
import os

import numpy as np
import pytest
import torch

import oracle
from miori_amd import ops, synth
from miori_amd._lib import MioriError
from tests._check import check_close
from tests.gpu_util import say, weights

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


@pytest.mark.parametrize("N,K,G", [(2048, 2048, 64), (8192, 2048, 64), (512, 2048, 32), (64, 8192, 128)])
def test_rmsnorm_gemv4(dev, N, K, G):
    say(f"rmsnorm_gemv4 N={N} K={K} G={G}")
    w, lin = weights(N, K, G, 4, seed=N + K, dev=dev)
    rng = np.random.default_rng(N)
    x = (rng.standard_normal(K) * 3).astype(np.float32)
    nw = synth.f32_to_bf16_bits((rng.standard_normal(K) * 0.2 + 1.0).astype(np.float32))
    y = torch.empty(N, dtype=torch.float32, device=dev)
    ops.rmsnorm_gemv4(torch.from_numpy(x).to(dev), ops.to_device_bits(nw, dev), lin.q, lin.s,
                      lin.b, y, N, K, group=G, eps=1e-5)
    torch.cuda.synchronize()
    h = oracle.rmsnorm_bf16(x, nw, 1e-5).reshape(1, K)
    ref = oracle.gemv_f64(w.q, w.s, w.b, h, 4, K, G, nthreads=NT)
    check_close(y.cpu().numpy().reshape(1, N), ref, f"rmsnorm_gemv4 {N}x{K}")


@pytest.mark.parametrize("N,K,G", [(2048, 7680, 64), (2048, 8192, 64), (2048, 2048, 32), (96, 512, 128)])
def test_silu_mul_gemv4(dev, N, K, G):
    say(f"silu_mul_gemv4 N={N} K={K} G={G}")
    w, lin = weights(N, K, G, 4, seed=N + K + 1, dev=dev)
    rng = np.random.default_rng(K)
    g = (rng.standard_normal(K) * 2).astype(np.float32)
    u = (rng.standard_normal(K)).astype(np.float32)
    y = torch.empty(N, dtype=torch.bfloat16, device=dev)
    ops.silu_mul_gemv4(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev), lin.q, lin.s,
                       lin.b, y, N, K, group=G)
    torch.cuda.synchronize()
    a = oracle.silu_mul_bf16(g, u).reshape(1, K)
    ref = oracle.gemv_f64(w.q, w.s, w.b, a, 4, K, G, nthreads=NT)
    check_close(ops.bits_of(y).reshape(1, N), ref, f"silu_mul_gemv4 {N}x{K}")


def test_fused_rejects_large_k(dev):
    w, lin = weights(16, 16384, 64, 4, seed=3, dev=dev)
    g = torch.zeros(16384, dtype=torch.float32, device=dev)
    y = torch.empty(16, dtype=torch.float32, device=dev)
    with pytest.raises(MioriError):
        ops.silu_mul_gemv4(g, g, lin.q, lin.s, lin.b, y, 16, 16384)


@pytest.mark.parametrize("N,K", [(2048, 2048), (2048, 7680)])
def test_silu_mul_gemv4_f32_out(dev, N, K):
    """fp32 outputs of small magnitude (gate and up uniform in +-1.5 / +-1):
    the 2-ulp bar then sees single bf16 rounding flips of the activation, so
    the transform's silu must track the CPU's expf and divide closely."""
    G = 64
    say(f"silu_mul_gemv4 f32 N={N} K={K}")
    w, lin = weights(N, K, G, 4, seed=N + 2 * K, dev=dev)
    rng = np.random.default_rng(K + 5)
    g = rng.uniform(-1.5, 1.5, K).astype(np.float32)
    u = rng.uniform(-1.0, 1.0, K).astype(np.float32)
    y = torch.empty(N, dtype=torch.float32, device=dev)
    ops.silu_mul_gemv4(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev), lin.q, lin.s,
                       lin.b, y, N, K, group=G)
    torch.cuda.synchronize()
    a = oracle.silu_mul_bf16(g, u).reshape(1, K)
    ref = oracle.gemv_f64(w.q, w.s, w.b, a, 4, K, G, nthreads=NT)
    check_close(y.cpu().numpy().reshape(1, N), ref, f"silu_mul_gemv4 f32 {N}x{K}")
