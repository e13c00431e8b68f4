"""CPU oracle for the quantized-matmul hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only as the checker. The product path
(``miori_amd``) never imports it and has no CPU fallback.

ctypes wrapper over ``oracle/_build/libmiori_oracle.so`` built from
``cpu_ref.c`` (plain-C restatement of the reference's src/cpu_ref.h:9-45 and
of its check loops src/main.cpp:73-84 and :594-601).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libmiori_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    if force or not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        lib = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_bf16_to_f32.restype = ctypes.c_float
        lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        lib.orc_f32_to_bf16_array.argtypes = [P, P, I]
        for name in ("orc_dequant4_elem", "orc_dequant8_elem"):
            f = getattr(lib, name)
            f.argtypes = [P, P, P, I, I, I, I]
            f.restype = ctypes.c_float
        for name in ("orc_dequant4_f32", "orc_dequant8_f32",
                     "orc_dequant4_bf16", "orc_dequant8_bf16"):
            getattr(lib, name).argtypes = [P, P, P, P, I, I, I]
        for name in ("orc_gemv4_f64", "orc_gemv8_f64"):
            getattr(lib, name).argtypes = [P, P, P, P, P, I, I, I, I, ctypes.c_int]
        for name in ("orc_gemv4_rows_f64", "orc_gemv8_rows_f64"):
            getattr(lib, name).argtypes = [P, P, P, P, P, I, I, I, I, I, I, ctypes.c_int]
        lib.orc_gemm_bf16_f64.argtypes = [P, P, P, I, I, I, P, I, ctypes.c_int]
        lib.orc_gemm_naive_f32.argtypes = [P, P, P, I, I, I, I, I, I]
        lib.orc_rmsnorm_bf16.argtypes = [P, P, P, I, ctypes.c_float]
        lib.orc_silu_mul_bf16.argtypes = [P, P, P, I]
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _check_q(q, s, b, bits, K, G):
    per_word = 32 // bits
    assert q.dtype == np.uint32 and q.shape[1] * per_word == K, (q.shape, K)
    assert s.dtype == np.uint16 and b.dtype == np.uint16
    assert s.shape == (q.shape[0], K // G) and b.shape == s.shape, (s.shape, K, G)


def bf16_to_f32(v: np.ndarray) -> np.ndarray:
    """src/cpu_ref.h:9-14, vectorised (bits << 16)."""
    return (np.asarray(v, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """src/cpu_ref.h:16-23 (RNE) through the C oracle."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    _load().orc_f32_to_bf16_array(_p(f), _p(out), f.size)
    return out


def dequant4_elem(q, s, b, n, k, K, G):
    _check_q(q, s, b, 4, K, G)
    return _load().orc_dequant4_elem(_p(q), _p(s), _p(b), n, k, K, G)


def dequant8_elem(q, s, b, n, k, K, G):
    _check_q(q, s, b, 8, K, G)
    return _load().orc_dequant8_elem(_p(q), _p(s), _p(b), n, k, K, G)


def dequant_f32(q, s, b, bits, K, G) -> np.ndarray:
    _check_q(q, s, b, bits, K, G)
    N = q.shape[0]
    out = np.empty((N, K), dtype=np.float32)
    fn = _load().orc_dequant4_f32 if bits == 4 else _load().orc_dequant8_f32
    fn(_p(q), _p(s), _p(b), _p(out), N, K, G)
    return out


def dequant_bf16(q, s, b, bits, K, G) -> np.ndarray:
    _check_q(q, s, b, bits, K, G)
    N = q.shape[0]
    out = np.empty((N, K), dtype=np.uint16)
    fn = _load().orc_dequant4_bf16 if bits == 4 else _load().orc_dequant8_bf16
    fn(_p(q), _p(s), _p(b), _p(out), N, K, G)
    return out


def gemv_f64(q, s, b, x, bits, K, G, nthreads: int = 1) -> np.ndarray:
    """y[M][N] fp64 per src/main.cpp:73-84; x is bf16 bits [M][K]."""
    _check_q(q, s, b, bits, K, G)
    x = np.ascontiguousarray(x.reshape(-1, K), dtype=np.uint16)
    M, N = x.shape[0], q.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    fn = _load().orc_gemv4_f64 if bits == 4 else _load().orc_gemv8_f64
    fn(_p(q), _p(s), _p(b), _p(x), _p(y), M, N, K, G, nthreads)
    return y


def gemv_rows_f64(q, s, b, x, bits, K, G, n0, n1, nthreads: int = 1) -> np.ndarray:
    """As gemv_f64 for output rows [n0, n1) only; other columns are left 0."""
    _check_q(q, s, b, bits, K, G)
    x = np.ascontiguousarray(x.reshape(-1, K), dtype=np.uint16)
    M, N = x.shape[0], q.shape[0]
    y = np.zeros((M, N), dtype=np.float64)
    fn = _load().orc_gemv4_rows_f64 if bits == 4 else _load().orc_gemv8_rows_f64
    fn(_p(q), _p(s), _p(b), _p(x), _p(y), M, N, K, G, n0, n1, nthreads)
    return y


def gemm_bf16_f64(A, B, rows=None, nthreads: int = 1) -> np.ndarray:
    """C[r][N] fp64 per src/main.cpp:594-601 for the selected rows of A."""
    A = np.ascontiguousarray(A, dtype=np.uint16)
    B = np.ascontiguousarray(B, dtype=np.uint16)
    M, K = A.shape
    N = B.shape[0]
    assert B.shape[1] == K
    rows = np.arange(M, dtype=np.int64) if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    C = np.empty((rows.size, N), dtype=np.float64)
    _load().orc_gemm_bf16_f64(_p(A), _p(B), _p(C), M, N, K, _p(rows), rows.size, nthreads)
    return C


def gemm_naive_f32(A, B, M, N, K, lda, ldb, ldc) -> np.ndarray:
    """C[M*ldc] fp32 per shaders/ops.metal:199-251 (sequential fp32 FMA chain
    over k), A and B given as flat bf16 bit arrays with row strides lda / ldb."""
    A = np.ascontiguousarray(A, dtype=np.uint16).ravel()
    B = np.ascontiguousarray(B, dtype=np.uint16).ravel()
    assert A.size >= (M - 1) * lda + K and B.size >= (N - 1) * ldb + K
    C = np.zeros(M * ldc, dtype=np.float32)
    _load().orc_gemm_naive_f32(_p(A), _p(B), _p(C), M, N, K, lda, ldb, ldc)
    return C


def rmsnorm_bf16(x, w, eps: float) -> np.ndarray:
    """bf16 bits of rmsnorm(x) * w per shaders/ops.metal:86-114 (one row)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    h = np.empty(x.size, dtype=np.uint16)
    _load().orc_rmsnorm_bf16(_p(x), _p(w), _p(h), x.size, eps)
    return h


def silu_mul_bf16(g, u) -> np.ndarray:
    """bf16 bits of silu(g) * u per shaders/ops.metal:129-139."""
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    a = np.empty(g.size, dtype=np.uint16)
    _load().orc_silu_mul_bf16(_p(g), _p(u), _p(a), g.size)
    return a
