"""GPU parity of the decode GEMVs (gemv4 / gemv8 / batched) against the oracle.

Reference behaviour: shaders/ops.metal:6-82 and shaders/batch.metal:145-236,
checked as src/main.cpp:44-87 does (fp64 sums of the CPU dequant times x),
with the benchmark's tolerance written in tests/_check.py.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from miori_amd import ops, synth
from miori_amd._lib import MioriError
from tests._check import check_close
from tests.gpu_util import acts, say, strided_rows, weights

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def _run(lin, x_dev, M, out_dtype):
    y = lin.gemv(x_dev, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return ops.bits_of(y).reshape(M, lin.N)


@pytest.mark.parametrize("N,K,G,odt", [
    (8192, 2048, 64, torch.bfloat16),   # the headline config
    (8192, 2048, 64, torch.float32),
    (512, 2048, 64, torch.float32),     # k/v_proj
    (2048, 8192, 64, torch.float32),    # down_proj: K split over 4 waves
    (300, 7680, 32, torch.float32),     # reference FFN width, ragged chunk count
    (64, 128, 32, torch.float32),       # tiny K: 4 active lanes
    (33, 4096, 128, torch.bfloat16),    # ragged N, group 128
    (7, 16384, 64, torch.float32),      # 2 chunks per lane
    (5, 32768, 64, torch.float32),      # largest K
    (33, 2048, 64, torch.bfloat16),     # lane-exchanged scales, ragged last block
    (1001, 1024, 32, torch.float32),    # lane-exchanged scales, two dwords per lane
])
def test_gemv4_parity(dev, N, K, G, odt):
    say(f"gemv4 N={N} K={K} G={G} out={odt}")
    w, lin = weights(N, K, G, 4, seed=N + K + G, dev=dev)
    x, xd = acts(1, K, seed=K + 1, dev=dev)
    y = _run(lin, xd, 1, odt)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, G, nthreads=NT)
    check_close(y, ref, f"gemv4 {N}x{K}")


def test_gemv4_reference_xfn(dev):
    """The reference test's activation x[k] = ((37k mod 101) - 50)/50
    (src/main.cpp:28) on a q_proj-shaped 2048x2048 matrix, group 32 as the
    reference model uses (config/m6.h:48)."""
    N = K = 2048
    G = 32
    say("gemv4 xfn 2048x2048 G=32")
    w, lin = weights(N, K, G, 4, seed=2, dev=dev)
    xf = ((np.arange(K) * 37) % 101 - 50).astype(np.float32) / np.float32(50.0)
    x = synth.f32_to_bf16_bits(xf).reshape(1, K)
    y = _run(lin, ops.to_device_bits(x, dev), 1, torch.float32)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, G, nthreads=NT)
    check_close(y, ref, "gemv4 xfn")


@pytest.mark.parametrize("bits", [4, 8])
def test_gemv_unpack_one_hot_exact(dev, bits):
    """s=1, b=0, x = e_k: y[n] must equal code(n, k) exactly, for every k of
    a 256-wide row (bit-exact unpacking through the GEMV path)."""
    N, K, G = 96, 256, 32
    say(f"gemv{bits} one-hot unpack")
    w = synth.quant_weights(N, K, G, bits, seed=77)
    ones = np.full((N, K // G), 0x3F80, dtype=np.uint16)
    zeros = np.zeros((N, K // G), dtype=np.uint16)
    q = ops.to_device_bits(w.q, dev)
    s = ops.to_device_bits(ones, dev)
    b = ops.to_device_bits(zeros, dev)
    deq = oracle.dequant_f32(w.q, ones, zeros, bits, K, G)
    fn = ops.gemv4 if bits == 4 else ops.gemv8
    for k in range(K):
        x = np.zeros((1, K), dtype=np.uint16)
        x[0, k] = 0x3F80
        y = torch.empty(N, dtype=torch.float32, device=dev)
        fn(q, s, b, ops.to_device_bits(x, dev), y, N, K, group=G)
        got = y.cpu().numpy()
        np.testing.assert_array_equal(got, deq[:, k], err_msg=f"k={k}")


@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 16, 32])
@pytest.mark.parametrize("N,K", [(2048, 2048), (512, 2048)])
def test_gemv4_batched_small_shapes(dev, M, N, K):
    G = 64
    say(f"gemv4_b M={M} N={N} K={K}")
    w, lin = weights(N, K, G, 4, seed=M * 31 + N, dev=dev)
    x, xd = acts(M, K, seed=M + 100, dev=dev)
    y = _run(lin, xd, M, torch.float32)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, 4, K, G, nthreads=NT)
    check_close(y, ref, f"gemv4_b M={M}")


@pytest.mark.parametrize("M", [4, 32])
@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192)])
def test_gemv4_batched_large_shapes(dev, M, N, K):
    G = 64
    say(f"gemv4_b M={M} N={N} K={K}")
    w, lin = weights(N, K, G, 4, seed=M * 7 + K, dev=dev)
    x, xd = acts(M, K, seed=M + 200, dev=dev)
    y = _run(lin, xd, M, torch.bfloat16)
    rows = strided_rows(N, 7)
    sub = synth.QuantWeights(np.ascontiguousarray(w.q[rows]), np.ascontiguousarray(w.s[rows]),
                             np.ascontiguousarray(w.b[rows]), 4, rows.size, K, G)
    ref = oracle.gemv_f64(sub.q, sub.s, sub.b, x, 4, K, G, nthreads=NT)
    check_close(y[:, rows], ref, f"gemv4_b M={M} {N}x{K}")


@pytest.mark.parametrize("bits,N,M", [(4, 2048, 4), (4, 8192, 2), (4, 4096, 3), (4, 8192, 4), (8, 16384, 2), (8, 8192, 4)])
def test_gemv4_batched_rows_equal_single(dev, bits, N, M):
    """Each batched row is the single-row product: bit-identical for M <= 4,
    the reference's guarantee (shaders/batch.metal:142-144), whatever the
    rows per wave (two to four rows of x take four weight rows per wave
    from N = 4096)."""
    K, G = 2048, 64
    say(f"gemv{bits}_b rows == gemv{bits} N={N} M={M}")
    w, lin = weights(N, K, G, bits, seed=5, dev=dev)
    x, xd = acts(M, K, seed=6, dev=dev)
    yb = lin.gemv(xd, torch.float32)
    for m in range(M):
        y1 = lin.gemv(xd[m:m + 1], torch.float32)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(yb[m].cpu().numpy(), y1[0].cpu().numpy())


@pytest.mark.parametrize("M", [1, 8, 32])
def test_gemv8_lm_head(dev, M):
    """Config: tied lm_head N=131072, K=2048, group 64; rows checked on a
    stride as the reference test does (every 997th there, src/main.cpp:74)."""
    N, K, G = 131072, 2048, 64
    say(f"gemv8 M={M} N={N}")
    w, lin = weights(N, K, G, 8, seed=88, dev=dev)
    x, xd = acts(M, K, seed=M + 300, dev=dev)
    y = _run(lin, xd, M, torch.bfloat16)
    rows = strided_rows(N, 997 if M > 1 else 97)
    sub_q, sub_s, sub_b = (np.ascontiguousarray(a[rows]) for a in (w.q, w.s, w.b))
    ref = oracle.gemv_f64(sub_q, sub_s, sub_b, x, 8, K, G, nthreads=NT)
    check_close(y[:, rows], ref, f"gemv8 M={M}")
    del lin
    torch.cuda.empty_cache()


@pytest.mark.parametrize("N,K,G", [(1000, 2048, 32), (64, 4096, 16), (31, 16384, 128)])
def test_gemv8_shapes(dev, N, K, G):
    say(f"gemv8 N={N} K={K} G={G}")
    w, lin = weights(N, K, G, 8, seed=N + G, dev=dev)
    x, xd = acts(1, K, seed=9, dev=dev)
    y = _run(lin, xd, 1, torch.float32)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, 8, K, G, nthreads=NT)
    check_close(y, ref, f"gemv8 {N}x{K}")


def test_gemv_rejects_bad_shapes(dev):
    w, lin = weights(16, 256, 64, 4, seed=1, dev=dev)
    x, xd = acts(1, 256, seed=1, dev=dev)
    y = torch.empty(16, dtype=torch.float32, device=dev)
    with pytest.raises(MioriError):
        ops.gemv4(lin.q, lin.s, lin.b, xd, y, 16, 256, group=48)
    with pytest.raises(ValueError):   # buffer too small for the shape
        ops.gemv4(lin.q, lin.s, lin.b, xd, y, 32, 256, group=64)
    with pytest.raises(MioriError):
        yb = torch.empty(33 * 16, dtype=torch.float32, device=dev)
        xb = torch.zeros(33 * 256, dtype=torch.bfloat16, device=dev)
        ops.gemv4_b(lin.q, lin.s, lin.b, xb, yb, 16, 256, 33, group=64)


@pytest.mark.parametrize("bits,M,N,K,G", [
    (4, 8, 1000, 2048, 32), (4, 24, 640, 4096, 128), (4, 5, 96, 1024, 64),
    (8, 12, 700, 2048, 32), (8, 32, 256, 4096, 128), (8, 6, 64, 512, 64),
])
def test_batched_skinny_groups(dev, bits, M, N, K, G):
    """The MFMA (skinny) batched path with every group size and ragged N."""
    say(f"gemv{bits}_b skinny M={M} N={N} K={K} G={G}")
    w, lin = weights(N, K, G, bits, seed=M * 13 + N + G, dev=dev)
    x, xd = acts(M, K, seed=M + 400, dev=dev)
    y = _run(lin, xd, M, torch.float32)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, bits, K, G, nthreads=NT)
    check_close(y, ref, f"gemv{bits}_b M={M} G={G}")


@pytest.mark.parametrize("bits,M,N,K,G", [
    (4, 6, 32784, 1024, 32), (4, 20, 32768, 2048, 128), (4, 32, 40000, 4096, 64),
    (8, 5, 32800, 1024, 32), (8, 12, 32768, 2048, 32), (8, 9, 33024, 512, 64),
    (8, 6, 33024, 2048, 32),
])
def test_batched_skinny_four_wave(dev, bits, M, N, K, G):
    """Vocabulary-sized N: the four-wave workgroups (two n-tiles up to M = 8,
    four above), every group size, ragged N and K from one to eight blocks
    per wave."""
    say(f"gemv{bits}_b four-wave M={M} N={N} K={K} G={G}")
    w, lin = weights(N, K, G, bits, seed=M * 7 + G, dev=dev)
    x, xd = acts(M, K, seed=M + 900, dev=dev)
    y = _run(lin, xd, M, torch.bfloat16)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, bits, K, G, nthreads=NT)
    check_close(y, ref, f"gemv{bits}_b four-wave M={M} G={G}")


@pytest.mark.parametrize("M,N,K,G", [
    (5, 32776, 2048, 64), (8, 32768, 1024, 128),
    (9, 40008, 1024, 128), (16, 32768, 2048, 128), (12, 32768, 4096, 128),
    (17, 32784, 2048, 64), (32, 50000, 1024, 64),
])
def test_gemv8_batched_persistent(dev, M, N, K, G):
    """8-bit, 5 <= M <= 32 at vocabulary-sized N: the persistent form (x in
    LDS once per CU, whole 16-row tiles over the full K per wave), with ragged
    N, one and two m-tiles, 16 to 64 blocks per tile and 16 or 32 of them in
    flight."""
    say(f"gemv8_b persistent M={M} N={N} K={K} G={G}")
    w, lin = weights(N, K, G, 8, seed=M * 5 + N, dev=dev)
    x, xd = acts(M, K, seed=M + 950, dev=dev)
    y = _run(lin, xd, M, torch.bfloat16)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, 8, K, G, nthreads=NT)
    check_close(y, ref, f"gemv8_b persistent M={M} N={N} K={K}")


@pytest.mark.parametrize("bits,M,N,K,G", [
    (4, 9, 2048, 8704, 64),     # K split in 4: 2176 k per workgroup (17 x 128)
    (8, 12, 1024, 8448, 32),    # K split in 4: 2112 k, rows padded to 2176 in LDS
    (4, 32, 8192, 2048, 64),    # two m-tiles, the whole 2048 k in LDS (128 KiB)
    (4, 32, 2048, 8192, 64),    # two m-tiles of a K split
    (8, 7, 3000, 2560, 64),     # 2560 k: five 512-element pieces
    (4, 13, 16400, 2048, 128),  # four n-tiles above M = 8 at N >= 16384
])
def test_batched_skinny_lds_x(dev, bits, M, N, K, G):
    """The x tile in LDS over each workgroup's K range: K splits whose range
    is no multiple of 512 (or of 128) elements, one and two m-tiles, against
    the oracle."""
    say(f"gemv{bits}_b LDS x M={M} N={N} K={K} G={G}")
    w, lin = weights(N, K, G, bits, seed=M * 3 + K, dev=dev)
    x, xd = acts(M, K, seed=M + 970, dev=dev)
    y = _run(lin, xd, M, torch.bfloat16)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, bits, K, G, nthreads=NT)
    check_close(y, ref, f"gemv{bits}_b LDS x M={M} N={N} K={K}")


def test_gemv8_batched_lds_x_fallback(dev):
    """8-bit vocabulary-sized form at K = 1280 (x rows of two and a half
    512-element pieces), with the oracle's result; a misaligned x is rejected
    by the entry point."""
    M, N, K, G = 7, 32768, 1280, 32
    say(f"gemv8_b LDS-x fallback N={N} K={K} G={G}")
    w, lin = weights(N, K, G, 8, seed=K + G, dev=dev)
    x, xd = acts(M, K, seed=31, dev=dev)
    y = _run(lin, xd, M, torch.bfloat16)
    ref = oracle.gemv_f64(w.q, w.s, w.b, x, 8, K, G, nthreads=NT)
    check_close(y, ref, f"gemv8_b M={M} N={N} K={K}")
    buf = torch.empty(M * K + 8, dtype=xd.dtype, device=dev)
    xm = buf[1:1 + M * K].view(M, K)
    with pytest.raises(MioriError):
        _run(lin, xm, M, torch.bfloat16)
