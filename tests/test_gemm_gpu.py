"""GPU parity of the prefill GEMMs and of the weight-cache dequant builders.

Reference behaviour: shaders/gemm_mpp.metal (dequant_tile + gemm_mpp) and
shaders/ops.metal:142-166, :754-779 (dequant4 / dequant8). The reference has
no CPU check of its MPP GEMM (only a 32- vs 64-row self-consistency test,
src/main.cpp:1403-1443); these tests check against the fp64 oracle
(src/main.cpp:594-601 loop) under the benchmark tolerance.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from miori_amd import ops, synth
from tests._check import check_close
from tests.gpu_util import say, strided_rows

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


@pytest.mark.parametrize("bits,N,K,G", [
    (4, 8192, 2048, 64), (4, 2048, 8192, 64), (4, 48, 256, 32), (4, 16, 512, 128),
    (8, 1000, 2048, 64), (8, 40, 512, 32), (8, 8, 256, 16),
])
def test_dequant_bit_exact(dev, bits, N, K, G):
    say(f"dequant{bits} N={N} K={K} G={G}")
    w = synth.quant_weights(N, K, G, bits, seed=N * bits + G)
    lin = ops.QuantLinear(w, dev)
    out = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    if bits == 4:
        ops.dequant4(lin.q, lin.s, lin.b, out, N, K, group=G)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ops.bits_of(out), oracle.dequant_bf16(w.q, w.s, w.b, 4, K, G))
        out2 = torch.empty_like(out)
        ops.dequant_tile(lin.q, lin.s, lin.b, out2, N, K, group=G)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ops.bits_of(out2), ops.bits_of(out))
    else:
        ops.dequant8(lin.q, lin.s, lin.b, out, N, K, group=G)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ops.bits_of(out), oracle.dequant_bf16(w.q, w.s, w.b, 8, K, G))


def _operands(M, N, K, seed, dev, G=64):
    w = synth.quant_weights(N, K, G, 4, seed=seed)
    Bbits = oracle.dequant_bf16(w.q, w.s, w.b, 4, K, G)
    A = synth.activations(M, K, seed=seed + 1)
    return w, Bbits, A


def _rows_for(M):
    if M <= 300:
        return np.arange(M, dtype=np.int64)
    return strided_rows(M, 37)


@pytest.mark.parametrize("M,K,N", [
    (256, 2048, 8192), (1024, 2048, 8192), (1472, 2048, 8192),
    (256, 8192, 2048), (1024, 8192, 2048), (1472, 8192, 2048),
    (256, 2048, 2560), (1024, 2048, 2560), (1472, 2048, 2560),
    (1, 64, 16), (23, 128, 80), (300, 192, 144), (64, 2048, 6144),
    (1500, 2048, 8208),                                                  # ragged 256x256 tiles
    (1400, 2048, 8000),                                                  # ragged 192x256 tiles
    (32, 2048, 2048), (17, 512, 96), (8, 2560, 256), (32, 8192, 512),   # skinny path
])
def test_gemm_bf16_parity(dev, M, K, N):
    say(f"gemm_bf16 M={M} K={K} N={N}")
    w, Bbits, A = _operands(M, N, K, seed=M + N + K, dev=dev)
    Ad = ops.to_device_bits(A, dev)
    Bd = ops.to_device_bits(Bbits, dev)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ops.gemm_mpp(Ad, Bd, C, M, N, K)
    torch.cuda.synchronize()
    rows = _rows_for(M)
    ref = oracle.gemm_bf16_f64(A, Bbits, rows, nthreads=NT)
    check_close(ops.bits_of(C)[rows], ref, f"gemm {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N,G", [
    (1024, 2048, 8192, 64), (1472, 8192, 2048, 64), (256, 2048, 2560, 64),
    (1472, 2048, 8192, 64), (1500, 2048, 8208, 64),   # bf16 side on 192x256 / 256x256 tiles
    (1400, 2048, 8000, 64),
    (1024, 2048, 2560, 64), (1000, 2048, 2608, 32), (1024, 2048, 8192, 128),  # 128x128 / G
    (32, 2048, 2048, 64), (32, 8192, 2048, 64), (100, 256, 48, 32), (64, 512, 128, 128),
    (32, 2048, 8192, 64), (9, 1024, 80, 32), (20, 2048, 512, 128),      # skinny path
])
def test_gemm_q4_fused_parity(dev, M, K, N, G):
    """Fused 4-bit GEMM: against the oracle, and against the two-step
    dequant_tile + gemm_mpp on the same operands. Both take the same B values
    (bf16_rne(q*s + b)); where the bf16 product runs on the 16x16x32
    producer/consumer kernel and the fused one on 32x32x16 MFMAs, the two
    differ only by fp32 rounding of the k sums, else bit for bit."""
    say(f"gemm_q4 M={M} K={K} N={N} G={G}")
    w, Bbits, A = _operands(M, N, K, seed=M * 3 + N, dev=dev, G=G)
    lin = ops.QuantLinear(w, dev)
    Ad = ops.to_device_bits(A, dev)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    ops.gemm_q4(Ad, lin.q, lin.s, lin.b, C, M, N, K, group=G)
    Bd = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    ops.dequant_tile(lin.q, lin.s, lin.b, Bd, N, K, group=G)
    C2 = torch.empty_like(C)
    ops.gemm_mpp(Ad, Bd, C2, M, N, K)
    torch.cuda.synchronize()
    rows = _rows_for(M)
    ref = oracle.gemm_bf16_f64(A, Bbits, rows, nthreads=NT)
    check_close(ops.bits_of(C)[rows], ref, f"gemm_q4 {M}x{K}x{N}", f32_tight=True)
    _agree(ops.bits_of(C), ops.bits_of(C2), f"gemm_q4 vs two-step {M}x{K}x{N}")


def _agree(a, b, what):
    """Two fp32 products of the same bf16 operands with different MFMA
    shapes: equal up to fp32 rounding of the k sums (2e-5 of the largest
    magnitude; the products' own error against fp64 is checked separately)."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    tol = 2e-5 * float(np.abs(b).max())
    err = float(np.abs(a - b).max())
    assert err <= tol, f"{what}: max |diff| {err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("m_small,m_big", [(23, 32), (40, 64)])
def test_gemm_tile_shape_consistency(dev, m_small, m_big):
    """The reference's test-mpp-tile property (src/main.cpp:1403-1443): the
    rows of a small-M product equal the same rows of a larger-M product.
    It holds within each kernel family here, M <= 32 (skinny MFMA kernel)
    and M > 32 (tiled GEMM); gemm_mpp32 and gemm_mpp are one entry point."""
    K, N = 2048, 6144
    say(f"gemm {m_small} vs {m_big} rows")
    w, Bbits, A = _operands(m_big, N, K, seed=4, dev=dev)
    Ad = ops.to_device_bits(A, dev)
    Bd = ops.to_device_bits(Bbits, dev)
    Cs = torch.empty((m_small, N), dtype=torch.float32, device=dev)
    Cb = torch.empty((m_big, N), dtype=torch.float32, device=dev)
    Cs2 = torch.empty((m_small, N), dtype=torch.float32, device=dev)
    ops.gemm_mpp32(Ad, Bd, Cs, m_small, N, K)
    ops.gemm_mpp(Ad, Bd, Cs2, m_small, N, K)
    ops.gemm_mpp(Ad, Bd, Cb, m_big, N, K)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(Cs.cpu().numpy(), Cs2.cpu().numpy())
    np.testing.assert_array_equal(Cs.cpu().numpy(), Cb[:m_small].cpu().numpy())


_CLASSIC = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
from miori_amd import ops
M, N, K = map(int, sys.argv[2:5])
A = torch.from_numpy(np.load(sys.argv[5])).cuda().view(torch.bfloat16)
B = torch.from_numpy(np.load(sys.argv[6])).cuda().view(torch.bfloat16)
C = torch.empty((M, N), dtype=torch.float32, device="cuda")
ops.gemm_mpp(A, B, C, M, N, K)
torch.cuda.synchronize()
np.save(sys.argv[7], C.cpu().numpy())
"""


@pytest.mark.parametrize("M,K,N", [(1024, 2048, 8192), (1472, 2048, 2560), (300, 8192, 2048),
                                   (1472, 8192, 2048)])  # the last on 192x128 tiles, split in 2
def test_gemm_producer_consumer_matches_classic(dev, tmp_path, M, K, N):
    """The eight-wave producer/consumer bf16 GEMM (the default for 256x128
    and 128x128 tiles, 16x16x32 MFMAs) agrees with the four-wave form on the
    same tiles (MIORI_GEMM_PC=0, 32x32x16 MFMAs, run in a child process: the
    switch is read once per process) up to fp32 rounding of the k sums."""
    import subprocess
    import sys

    say(f"gemm producer/consumer vs classic M={M} K={K} N={N}")
    w, Bbits, A = _operands(M, N, K, seed=M + 5 * N, dev=dev)
    Ad = ops.to_device_bits(A, dev)
    Bd = ops.to_device_bits(Bbits, dev)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    ops.gemm_mpp(Ad, Bd, C, M, N, K)
    torch.cuda.synchronize()
    fa, fb, fc = tmp_path / "a.npy", tmp_path / "b.npy", tmp_path / "c.npy"
    np.save(fa, A.view(np.int16))
    np.save(fb, Bbits.view(np.int16))
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, MIORI_GEMM_PC="0")
    r = subprocess.run([sys.executable, "-c", _CLASSIC, root, str(M), str(N), str(K), str(fa),
                        str(fb), str(fc)], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    _agree(C.cpu().numpy(), np.load(fc), f"producer/consumer vs four-wave {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(1472, 2048, 8192), (1500, 2048, 8208), (2048, 2048, 8192)])
def test_gemm_eight_wave_matches_producer_consumer(dev, tmp_path, M, K, N):
    """The eight-wave tall-tile kernel (192x256 and 256x256 tiles, the
    default at these shapes) runs the producer/consumer kernel's 16x16x32
    MFMA order, so its products equal those of the 256x128 producer/consumer
    tiles (MIORI_GEMM_TILE=0, run in a child process: the switch is read
    once per process) bit for bit, ragged edges included."""
    import subprocess
    import sys

    say(f"gemm eight-wave vs producer/consumer M={M} K={K} N={N}")
    w, Bbits, A = _operands(M, N, K, seed=M + 7 * N, dev=dev)
    Ad = ops.to_device_bits(A, dev)
    Bd = ops.to_device_bits(Bbits, dev)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    ops.gemm_mpp(Ad, Bd, C, M, N, K)
    torch.cuda.synchronize()
    fa, fb, fc = tmp_path / "a.npy", tmp_path / "b.npy", tmp_path / "c.npy"
    np.save(fa, A.view(np.int16))
    np.save(fb, Bbits.view(np.int16))
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, MIORI_GEMM_TILE="0", MIORI_GEMM_SPLIT="1")
    r = subprocess.run([sys.executable, "-c", _CLASSIC, root, str(M), str(N), str(K), str(fa),
                        str(fb), str(fc)], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    np.testing.assert_array_equal(C.cpu().numpy().view(np.uint32), np.load(fc).view(np.uint32))

