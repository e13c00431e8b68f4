"""GPU check of the shader-clock sampler (miori_diag_clock_sample, a
diagnostic with no counterpart in the reference): both counters advance, the
samples are the requested wall-clock gap apart, and the clock they imply
lies between 0.3 and 3 GHz (MI355X's peak engine clock is 2.4 GHz), alone
and beside a GEMM on another stream."""
import ctypes

import numpy as np
import pytest
import torch

from miori_amd import _lib, ops
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def _sample(dev, n, gap, stream):
    buf = torch.zeros(2 * n, dtype=torch.int64, device=dev)
    khz = ctypes.c_uint32(0)
    _lib.call("miori_diag_clock_sample", ctypes.c_void_p(buf.data_ptr()), n, gap,
              ctypes.byref(khz), ctypes.c_void_p(stream.cuda_stream))
    return buf, khz


def _check(buf, khz, n, gap):
    s = buf.cpu().numpy().view(np.uint64).reshape(n, 2).astype(np.float64)
    dc, dr = np.diff(s[:, 0]), np.diff(s[:, 1])
    assert khz.value > 0
    assert np.all(dc > 0) and np.all(dr >= gap), "counters must advance by at least the gap"
    ghz = (s[-1, 0] - s[0, 0]) / (s[-1, 1] - s[0, 1]) * khz.value * 1e3 / 1e9
    assert 0.3 < ghz < 3.0, ghz
    return ghz


def test_clock_sampler_alone(dev):
    n, gap = 256, 100
    say(f"clock sampler alone n={n} gap={gap}")
    st = torch.cuda.current_stream()
    buf, khz = _sample(dev, n, gap, st)
    torch.cuda.synchronize()
    _check(buf, khz, n, gap)


def test_clock_sampler_beside_gemm(dev):
    M, N, K = 1024, 2048, 2048
    n, gap = 400, 50
    say(f"clock sampler beside gemm_bf16 {M}x{N}x{K}")
    A = torch.randn(M, K, device=dev).to(torch.bfloat16)
    B = torch.randn(N, K, device=dev).to(torch.bfloat16)
    C = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ops.gemm_mpp(A, B, C, M, N, K)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=dev)
    buf, khz = _sample(dev, n, gap, side)
    for _ in range(20):
        ops.gemm_mpp(A, B, C, M, N, K)
    torch.cuda.synchronize()
    _check(buf, khz, n, gap)
    ref = A.float() @ B.float().t()
    assert ((C.float() - ref).abs().max() / ref.abs().max()).item() < 1e-2


def test_clock_sampler_rejects_more_than_two_seconds(dev):
    # the bound is 2 s at the device's own wall-clock rate: 2^20 samples 1 ms
    # apart is far over it on any part
    khz = ctypes.c_uint32(0)
    say("clock sampler bound")
    rc = _lib.status("miori_diag_clock_sample", ctypes.c_void_p(1 << 20), 1 << 20, 10**6,
                     ctypes.byref(khz), None)
    assert rc == -2


def test_gemv_timeline_matches_gemv4(dev):
    """The stamped diagnostic build computes the headline GEMV bit-identically
    to miori_gemv_q4, and every wave's stamps are in order (entry <= loads
    landed <= arithmetic done <= stores complete) and within the launch."""
    from tests.gpu_util import acts, weights
    N, K, G = 8192, 2048, 64
    say(f"gemv4 timeline N={N} K={K}")
    w, lin = weights(N, K, G, 4, seed=77, dev=dev)
    _, xd = acts(1, K, seed=78, dev=dev)
    y0 = torch.empty(N, dtype=torch.bfloat16, device=dev)
    y1 = torch.empty(N, dtype=torch.bfloat16, device=dev)
    ops.gemv4(lin.q, lin.s, lin.b, xd, y0, N, K, group=G)
    st = ops.gemv4_timeline(lin.q, lin.s, lin.b, xd, y1, N, K, group=G)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    s = st.cpu().numpy()
    assert s.shape == (N // 16 * 4, 4)
    assert np.all(s > 0)
    assert np.all(np.diff(s, axis=1) >= 0), "stamps out of order"
    # the whole launch spans well under a millisecond (100 MHz ticks)
    assert s[:, 3].max() - s[:, 0].min() < 100_000
