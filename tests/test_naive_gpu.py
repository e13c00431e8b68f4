"""GPU parity of the gemm_naive fallback (shaders/ops.metal:199-251 behind
src/ops.h:30-32) against the oracle's sequential fp32 FMA chain, bit for bit:
both evaluate the same k-ordered chain of exact bf16 products. The first case
is the reference's own test-gemm (src/main.cpp:578-602), recorded there as
max_abs 0 (docs/REGRESSION.md:12)."""
import numpy as np
import pytest
import torch

import oracle
from miori_amd import ops, synth
from miori_amd._lib import MioriError
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def _run(dev, a_bits, b_bits, M, N, K, lda, ldb, ldc, aoff=0, boff=0, coff=0):
    A = ops.to_device_bits(a_bits, dev)
    B = ops.to_device_bits(b_bits, dev)
    C = torch.full(((coff // 4) + M * ldc,), -7.0, dtype=torch.float32, device=dev)
    ops.gemm_naive(A, B, C, M, N, K, lda, ldb, ldc, aoff=aoff, boff=boff, coff=coff)
    torch.cuda.synchronize()
    return C.cpu().numpy()[coff // 4:]


def test_reference_test_gemm(dev):
    M, N, K, lda, ldb, ldc = 4, 8, 32, 64, 32, 16
    say("gemm_naive reference test-gemm case")
    a = synth.f32_to_bf16_bits(np.sin(np.arange(M * lda, dtype=np.float32) * np.float32(0.13)))
    b = synth.f32_to_bf16_bits(np.cos(np.arange(N * ldb, dtype=np.float32) * np.float32(0.17)))
    got = _run(dev, a, b, M, N, K, lda, ldb, ldc).reshape(M, ldc)
    ref = oracle.gemm_naive_f32(a, b, M, N, K, lda, ldb, ldc).reshape(M, ldc)
    assert np.abs(got[:, :N] - ref[:, :N]).max() == 0.0  # the reference records max_abs 0
    assert np.all(got[:, N:] == -7.0)  # padding columns untouched


@pytest.mark.parametrize("M,N,K,lda,ldb,ldc", [
    (1, 16, 2048, 2048, 2048, 16),      # gate_proj N=16, one token
    (128, 16, 2048, 2048, 2048, 16),    # gate_proj over a 128-token prefill chunk
    (8, 1000, 2048, 2048, 2048, 1000),  # batch lm_head-like, ragged N, 8-row tile
    (12, 1000, 2048, 2048, 2048, 1000), # 16-row tile, ragged N and M
    (37, 53, 77, 80, 100, 60),          # ragged everything, strided
    (16, 300, 96, 96, 96, 304),         # M exactly one small tile
    (70, 130, 200, 200, 256, 130),      # several tiles in both directions
    (32, 700, 2048, 2048, 2048, 700),   # batch lm_head-like at M = 32 (32 x 256 tiles)
    (24, 1000, 512, 512, 512, 1000),    # 32-row tile, 16-byte loads, ragged N and M
    (17, 257, 100, 104, 100, 260),      # 32-row tile, ragged and strided
    (8, 600, 2048, 2048, 2048, 600),    # 8-row tile (M <= 8)
    (3, 300, 90, 96, 90, 300),          # 8-row tile, ragged K and strides (element loads)
    (12, 300, 90, 96, 90, 300),         # 16x256 tile, element loads (K % 8 != 0)
    (5, 20, 100, 104, 100, 20),         # 16x16 tile (N <= 32), element loads
])
def test_naive_shapes_bit_exact(dev, M, N, K, lda, ldb, ldc):
    say(f"gemm_naive M={M} N={N} K={K} lda={lda} ldb={ldb} ldc={ldc}")
    a = synth.activations(M, lda, seed=M + K).ravel()
    b = synth.activations(N, ldb, seed=N + K + 1).ravel()
    got = _run(dev, a, b, M, N, K, lda, ldb, ldc).reshape(M, ldc)
    ref = oracle.gemm_naive_f32(a, b, M, N, K, lda, ldb, ldc).reshape(M, ldc)
    np.testing.assert_array_equal(got[:, :N], ref[:, :N])


def test_naive_byte_offsets(dev):
    """aoff / boff / coff select a sub-buffer, as the reference's encoder offsets do."""
    M, N, K, lda, ldb, ldc = 6, 20, 64, 64, 64, 20
    aoff, boff, coff = 2 * 64 * 3, 2 * 128, 4 * 40
    a = synth.activations(M + 3, lda, seed=11).ravel()
    b = synth.activations(N + 2, ldb, seed=12).ravel()
    got = _run(dev, a, b, M, N, K, lda, ldb, ldc, aoff, boff, coff).reshape(M, ldc)
    ref = oracle.gemm_naive_f32(a[aoff // 2:], b[boff // 2:], M, N, K, lda, ldb, ldc).reshape(M, ldc)
    np.testing.assert_array_equal(got, ref)


def test_naive_rejects_bad_args(dev):
    A = torch.zeros(64, dtype=torch.bfloat16, device=dev)
    C = torch.zeros(64, dtype=torch.float32, device=dev)
    with pytest.raises(MioriError):
        ops.gemm_naive(A, A, C, 2, 2, 32, 16, 32, 2)   # lda < K
    with pytest.raises(ValueError):
        ops.gemm_naive(A, A, C, 4, 4, 32, 32, 32, 4)   # A too small for the shape
