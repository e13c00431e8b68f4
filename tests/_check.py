"""Tolerance checks shared by the parity tests.

The bar (from the benchmark definition): against the fp64 CPU reference,
max|delta| <= 1e-2 * max|ref| and at least 99.9% of elements within 2 bf16
ulp of the reference value. fp32 outputs must in addition be fp32-accurate
(max|delta| <= 1e-4 * max|ref|), because every operand the kernels multiply
is exact and only the fp32 sums round.
"""
from __future__ import annotations

import numpy as np


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (8 significant bits)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    a = np.where(a < 2.0 ** -126, 2.0 ** -126, a)
    e = np.floor(np.log2(a))
    return 2.0 ** (e - 7)


def as_f64(out: np.ndarray) -> np.ndarray:
    """Device output (fp32 array or bf16 bits as uint16) -> float64."""
    out = np.asarray(out)
    if out.dtype == np.uint16:
        return (out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return out.astype(np.float64)


def check_close(out, ref, what: str = "", f32_tight: bool | None = None) -> dict:
    out = np.asarray(out)
    is_bf16 = out.dtype == np.uint16
    o = as_f64(out)
    ref = np.asarray(ref, dtype=np.float64)
    assert o.shape == ref.shape, (what, o.shape, ref.shape)
    assert np.all(np.isfinite(o)), f"{what}: non-finite outputs"
    d = np.abs(o - ref)
    mref = float(np.max(np.abs(ref))) if ref.size else 0.0
    maxd = float(d.max()) if d.size else 0.0
    within = float(np.mean(d <= 2.0 * bf16_ulp(ref))) if d.size else 1.0
    stats = {"max_abs": maxd, "max_ref": mref, "frac_2ulp": within}
    assert maxd <= 1e-2 * mref + 1e-30, f"{what}: max|d|={maxd:.3g} > 1e-2*{mref:.3g}"
    assert within >= 0.999, f"{what}: only {within:.5f} within 2 bf16 ulp"
    if f32_tight is None:
        f32_tight = not is_bf16
    if f32_tight:
        assert maxd <= 1e-4 * mref + 1e-30, f"{what}: fp32 max|d|={maxd:.3g} > 1e-4*{mref:.3g}"
    return stats
