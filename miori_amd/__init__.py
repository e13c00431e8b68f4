"""miori_amd: MI355X (gfx950) quantized-matmul hot path of Miori.

The kernels live in libmiori_hip.so (miori_amd/csrc, C ABI in
include/miori_hip.h); ``miori_amd.ops`` mirrors the reference's src/ops.h
wrappers on top of it, ``miori_amd.synth`` draws seeded synthetic operands.
"""
from . import synth  # noqa: F401

__all__ = ["synth", "ops", "build"]
