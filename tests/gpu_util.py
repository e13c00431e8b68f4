"""Helpers for the GPU parity tests: seeded operands on host and device."""
from __future__ import annotations

import sys

import numpy as np
import torch

from miori_amd import ops, synth


def say(*a):
    """Name the case on stdout before a GPU step (flushed)."""
    print(*a, flush=True)
    sys.stdout.flush()


def out_bits(y: torch.Tensor) -> np.ndarray:
    return ops.bits_of(y)


def weights(N, K, G, bits, seed, dev):
    w = synth.quant_weights(N, K, G, bits, seed=seed)
    return w, ops.QuantLinear(w, dev)


def acts(M, K, seed, dev):
    x = synth.activations(M, K, seed=seed)
    return x, ops.to_device_bits(x, dev)


def strided_rows(N, step):
    rows = np.unique(np.concatenate([np.arange(0, N, step), np.arange(max(0, N - 5), N)]))
    return rows.astype(np.int64)
