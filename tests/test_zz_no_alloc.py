"""miori_gemm_q4_static, the allocation-free fused 4-bit GEMM: called through
the C ABI, its output must equal miori_gemm_q4's bit for bit (the same
kernels and split, with the partials in the fixed per-GPU scratch array),
on two calls in a row, the second smaller; a shape whose partials exceed the
array is rejected before anything is enqueued."""
import ctypes

import numpy as np
import pytest
import torch

from miori_amd import _lib, ops
from tests.gpu_util import say

pytestmark = pytest.mark.gpu

MIORI_E_SCRATCH = -6


def _quant(N, K, gen, dev):
    q = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), dtype=torch.int32, device=dev,
                      generator=gen)
    s = (0.001 + 0.009 * torch.rand(N, K // 64, device=dev, generator=gen)).to(torch.bfloat16)
    b = (-8.0 * s.float() + 1e-3 * torch.randn(N, K // 64, device=dev, generator=gen)).to(
        torch.bfloat16)
    return q, s, b


def _call(name, A, q, s, b, C, M, N, K):
    stream = torch.cuda.current_stream().cuda_stream
    od = _lib.MIORI_BF16 if C.dtype == torch.bfloat16 else _lib.MIORI_F32
    return _lib.status(name, A.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(),
                       C.data_ptr(), M, N, K, 64, od, stream)


# (M, N, K): split-K on the skinny path (M > 8, K = 8192: 4 splits), then on
# the MFMA GEMM (M = 1024, K = 8192), then a smaller skinny product
SEQUENCE = [(32, 8192, 8192), (1024, 2048, 8192), (16, 2048, 8192)]


def test_static_matches_allocating_entry(dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    for M, N, K in SEQUENCE:
        say(f"gemm_q4_static M={M} N={N} K={K}")
        q, s, b = _quant(N, K, gen, dev)
        A = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        want = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        got = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        assert _call("miori_gemm_q4", A, q, s, b, want, M, N, K) == 0
        assert _call("miori_gemm_q4_static", A, q, s, b, got, M, N, K) == 0
        torch.cuda.synchronize()
        w, g = ops.bits_of(want), ops.bits_of(got)
        assert np.all(np.isfinite(w))
        np.testing.assert_array_equal(g.view(np.uint32), w.view(np.uint32),
                                      err_msg=f"M={M} N={N} K={K}")


def test_static_rejects_partials_beyond_scratch(dev):
    say("gemm_q4_static oversize rejection")
    gen = torch.Generator(device=dev)
    gen.manual_seed(12)
    M, N, K = 32, 131072, 8192           # 4 x 32 x 131072 x 4 B = 64 MiB of partials
    q, s, b = _quant(N, K, gen, dev)
    A = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
    C = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    assert _call("miori_gemm_q4_static", A, q, s, b, C, M, N, K) == MIORI_E_SCRATCH
    torch.cuda.synchronize()
    assert bool(torch.all(C == 7.0)), "nothing may be written when the scratch is too small"
    msg = _lib.load().miori_status_string(MIORI_E_SCRATCH)
    assert b"scratch" in msg
