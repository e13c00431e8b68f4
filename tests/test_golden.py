"""The committed fixtures (tests/golden/golden.npz, made by make_golden.py):
the CPU oracle and the seeded generator must reproduce them exactly, and the
GPU kernels must match them (dequant bit-exact, products within tolerance)."""
import os
import re

import numpy as np
import pytest

import oracle
from miori_amd import synth
from tests._check import check_close

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
G = np.load(PATH, allow_pickle=False)
GEMV_KEYS = sorted({k[: k.rindex("_")] for k in G.files if k.startswith("q")})


def _parse(key):
    bits, N, K, grp, M = map(int, re.match(r"q(\d+)_n(\d+)_k(\d+)_g(\d+)_m(\d+)", key).groups())
    return bits, N, K, grp, M


@pytest.mark.parametrize("key", GEMV_KEYS)
def test_oracle_reproduces_fixture(key):
    bits, N, K, grp, M = _parse(key)
    q, s, b, x = (G[key + s_] for s_ in ("_q", "_s", "_b", "_x"))
    np.testing.assert_array_equal(oracle.gemv_f64(q, s, b, x, bits, K, grp), G[key + "_y"])
    np.testing.assert_array_equal(oracle.dequant_bf16(q, s, b, bits, K, grp), G[key + "_deq"])


def test_generator_reproduces_fixture_inputs():
    w = synth.quant_weights(64, 256, 32, 4, seed=101)
    np.testing.assert_array_equal(w.q, G["q4_n64_k256_g32_m1_q"])
    np.testing.assert_array_equal(w.s, G["q4_n64_k256_g32_m1_s"])
    np.testing.assert_array_equal(synth.activations(1, 256, seed=1101), G["q4_n64_k256_g32_m1_x"])


def test_reference_gemm_fixture():
    np.testing.assert_array_equal(oracle.gemm_bf16_f64(G["gemm_ref_A"], G["gemm_ref_B"]), G["gemm_ref_C"])
    np.testing.assert_array_equal(
        oracle.gemm_bf16_f64(G["gemm_q4_A"], oracle.dequant_bf16(G["gemm_q4_q"], G["gemm_q4_s"],
                                                                 G["gemm_q4_b"], 4, 128, 64)),
        G["gemm_q4_C"])


@pytest.mark.gpu
@pytest.mark.parametrize("key", GEMV_KEYS)
def test_gpu_matches_fixture(dev, key):
    import torch

    from miori_amd import ops

    bits, N, K, grp, M = _parse(key)
    print(f"golden {key}", flush=True)
    q, s, b = (ops.to_device_bits(G[key + s_], dev) for s_ in ("_q", "_s", "_b"))
    x = ops.to_device_bits(G[key + "_x"], dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    if M == 1:
        (ops.gemv4 if bits == 4 else ops.gemv8)(q, s, b, x, y, N, K, group=grp)
    else:
        (ops.gemv4_b if bits == 4 else ops.gemv8_b)(q, s, b, x, y, N, K, M, group=grp)
    out = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    (ops.dequant4 if bits == 4 else ops.dequant8)(q, s, b, out, N, K, group=grp)
    torch.cuda.synchronize()
    check_close(y.cpu().numpy(), G[key + "_y"], key)
    np.testing.assert_array_equal(ops.bits_of(out), G[key + "_deq"])


@pytest.mark.gpu
def test_gpu_gemm_fixtures(dev):
    import torch

    from miori_amd import ops

    print("golden gemm", flush=True)
    # the reference test-gemm shape needs K % 64 == 0 here: pad K 32 -> 64 with zeros
    A = np.zeros((4, 64), dtype=np.uint16)
    A[:, :32] = G["gemm_ref_A"]
    B = np.zeros((16, 64), dtype=np.uint16)
    B[:8, :32] = G["gemm_ref_B"]
    C = torch.empty((4, 16), dtype=torch.float32, device=dev)
    ops.gemm_mpp(ops.to_device_bits(A, dev), ops.to_device_bits(B, dev), C, 4, 16, 64)
    Cq = torch.empty((20, 48), dtype=torch.float32, device=dev)
    ops.gemm_q4(ops.to_device_bits(G["gemm_q4_A"], dev), ops.to_device_bits(G["gemm_q4_q"], dev),
                ops.to_device_bits(G["gemm_q4_s"], dev), ops.to_device_bits(G["gemm_q4_b"], dev),
                Cq, 20, 48, 128, group=64)
    torch.cuda.synchronize()
    check_close(C.cpu().numpy()[:, :8], G["gemm_ref_C"], "test-gemm operands")
    check_close(Cq.cpu().numpy(), G["gemm_q4_C"], "fused q4 fixture")
