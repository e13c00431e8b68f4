"""Seeded synthetic inputs for the quantized-matmul hot path.

The reference tests run on real model weights (src/main.cpp:44-87), which are
not available here, so every test and benchmark draws its operands from this
generator: splitmix64 streams (one per tensor, seeded from a config seed and a
tensor index), uniforms from the top 53 bits, normals by Box-Muller. The
distributions are the ones the benchmark configurations name:

* 4-bit weights (MLX affine, src/cpu_ref.h:25-34): nibbles uniform 0..15,
  packed 8 per uint32 little-endian along K; per group of G along K a bf16
  scale ~ U(0.001, 0.01) and a bf16 bias = -8*scale + N(0, 1e-3).
* 8-bit weights (src/cpu_ref.h:36-45): codes uniform 0..255, 4 per uint32;
  scale ~ U(1e-4, 1e-3), bias = -128*scale.
* activations: bf16 ~ N(0, 1).

bf16 values are rounded from fp32 with round-to-nearest-even, the rounding of
src/cpu_ref.h:16-23. Everything is numpy on the host; callers move the arrays
to the device themselves.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
BASE_SEED = 0x4D494F52  # "MIOR"


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of splitmix64 started at state ``seed``."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + _GOLDEN * np.arange(1, n + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    """U[0, 1) doubles from the top 53 bits of splitmix64."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, n: int) -> np.ndarray:
    """N(0, 1) doubles by Box-Muller over pairs of uniforms."""
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n]


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (no NaN special case)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    return ((u >> np.uint64(16)) & np.uint64(0xFFFF)).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def random_words(seed: int, n: int) -> np.ndarray:
    """n uniformly random uint32 words (every nibble / byte uniform)."""
    return (splitmix64(seed, n) >> np.uint64(32)).astype(np.uint32)


@dataclass
class QuantWeights:
    """One affine-quantized weight matrix W[N][K] in the MLX layout."""
    q: np.ndarray   # uint32 [N][K*bits/32]
    s: np.ndarray   # bf16 bits uint16 [N][K/G]
    b: np.ndarray   # bf16 bits uint16 [N][K/G]
    bits: int
    N: int
    K: int
    G: int

    @property
    def nbytes(self) -> int:
        return self.q.nbytes + self.s.nbytes + self.b.nbytes


def quant_weights(N: int, K: int, G: int = 64, bits: int = 4, seed: int = BASE_SEED) -> QuantWeights:
    """Seeded MLX-affine weights with the benchmark distributions."""
    assert bits in (4, 8) and K % G == 0 and K % 32 == 0
    ng = K // G
    words = N * K * bits // 32
    q = random_words(seed * 4 + 1, words).reshape(N, K * bits // 32)
    if bits == 4:
        sc = 0.001 + 0.009 * uniform(seed * 4 + 2, N * ng)
        s = f32_to_bf16_bits(sc.astype(np.float32))
        sf = bf16_bits_to_f32(s).astype(np.float64)
        bi = -8.0 * sf + 1e-3 * normal(seed * 4 + 3, N * ng)
        b = f32_to_bf16_bits(bi.astype(np.float32))
    else:
        sc = 1e-4 + 9e-4 * uniform(seed * 4 + 2, N * ng)
        s = f32_to_bf16_bits(sc.astype(np.float32))
        sf = bf16_bits_to_f32(s)
        b = f32_to_bf16_bits((np.float32(-128.0) * sf).astype(np.float32))
    return QuantWeights(q=q, s=s.reshape(N, ng), b=b.reshape(N, ng), bits=bits, N=N, K=K, G=G)


def activations(M: int, K: int, seed: int = BASE_SEED + 7) -> np.ndarray:
    """bf16 bits [M][K] ~ N(0, 1)."""
    return f32_to_bf16_bits(normal(seed, M * K).astype(np.float32)).reshape(M, K)
