"""Write tests/golden/golden.npz: small seeded cases with the oracle's outputs.

    python tests/golden/make_golden.py

The reference ships no golden vectors (its kernel tests read real model
weights and print errors without asserting, src/main.cpp:44-87), so these
fixtures are produced by the restated CPU oracle (oracle/cpu_ref.c) on the
in-repo seeded generator, plus the reference test-gemm operands
(src/main.cpp:578-602). They pin the oracle and the generator against
future changes and give the GPU tests fixed expected outputs.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from miori_amd import synth  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def cases():
    d = {}
    for bits, N, K, G, M, seed in [(4, 64, 256, 32, 1, 101), (4, 64, 256, 64, 3, 102),
                                   (4, 48, 512, 128, 2, 103), (8, 64, 256, 32, 1, 104),
                                   (8, 40, 512, 64, 4, 105)]:
        w = synth.quant_weights(N, K, G, bits, seed=seed)
        x = synth.activations(M, K, seed=seed + 1000)
        key = f"q{bits}_n{N}_k{K}_g{G}_m{M}"
        d[key + "_q"] = w.q
        d[key + "_s"] = w.s
        d[key + "_b"] = w.b
        d[key + "_x"] = x
        d[key + "_y"] = oracle.gemv_f64(w.q, w.s, w.b, x, bits, K, G)
        d[key + "_deq"] = oracle.dequant_bf16(w.q, w.s, w.b, bits, K, G)
    # the reference test-gemm operands: M=4, N=8, K=32, lda=64, ldb=32
    M, N, K, lda, ldb = 4, 8, 32, 64, 32
    a = synth.f32_to_bf16_bits(np.sin(np.arange(M * lda, dtype=np.float32) * np.float32(0.13)))
    b = synth.f32_to_bf16_bits(np.cos(np.arange(N * ldb, dtype=np.float32) * np.float32(0.17)))
    A = np.ascontiguousarray(a.reshape(M, lda)[:, :K])
    B = np.ascontiguousarray(b.reshape(N, ldb)[:, :K])
    d["gemm_ref_A"] = A
    d["gemm_ref_B"] = B
    d["gemm_ref_C"] = oracle.gemm_bf16_f64(A, B)
    # a GEMM on dequantised 4-bit weights (the fused path's operands)
    w = synth.quant_weights(48, 128, 64, 4, seed=106)
    A2 = synth.activations(20, 128, seed=107)
    B2 = oracle.dequant_bf16(w.q, w.s, w.b, 4, 128, 64)
    d["gemm_q4_q"], d["gemm_q4_s"], d["gemm_q4_b"] = w.q, w.s, w.b
    d["gemm_q4_A"] = A2
    d["gemm_q4_C"] = oracle.gemm_bf16_f64(A2, B2)
    return d


if __name__ == "__main__":
    np.savez_compressed(OUT, **cases())
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")
