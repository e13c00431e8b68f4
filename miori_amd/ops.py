"""Host-side mirror of the reference's hot-path op wrappers (src/ops.h).

Each function keeps the name and argument meaning of its src/ops.h
counterpart; the Metal (device, encoder, buffer + byte offset) arguments
become device tensors (a tensor view carries its own offset) and the
optional ``stream`` (default: torch's current stream). Like the reference
wrappers they only enqueue work; call ``sync()`` for the blocking
``Metal::submit(cb, wait=true)`` (src/metal.cpp:56-59).

The output dtype follows ``y`` / ``C``: torch.float32 is the reference's
``device float*`` output, torch.bfloat16 the RNE-rounded bf16 output.
Errors raise ``MioriError`` (a RuntimeError), the reference's error
convention (src/metal.cpp:31-37). Before anything is launched the buffer
sizes are checked against the shapes, so a wrong shape is an exception on
the host, never an out-of-bounds access on the device.

Torch is used for device memory and streams only; all arithmetic runs in
libmiori_hip.so.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import MIORI_BF16, MIORI_F32, MioriError  # noqa: F401


def _stream(stream):
    if stream is None:
        return ctypes_stream(torch.cuda.current_stream())
    if isinstance(stream, torch.cuda.Stream):
        return ctypes_stream(stream)
    return stream


def ctypes_stream(s: torch.cuda.Stream):
    return s.cuda_stream


def _ptr(t: torch.Tensor, name: str, min_bytes: int) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor (got {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    have = t.numel() * t.element_size()
    if have < min_bytes:
        raise ValueError(f"{name} holds {have} bytes, the shape needs {min_bytes}")
    return t.data_ptr()


def _out_dtype(y: torch.Tensor) -> int:
    if y.dtype == torch.float32:
        return MIORI_F32
    if y.dtype == torch.bfloat16:
        return MIORI_BF16
    raise ValueError(f"output dtype must be float32 or bfloat16, got {y.dtype}")


def _qargs(q, s, b, N, K, group, bits):
    return (_ptr(q, "q", N * K * bits // 8),
            _ptr(s, "scales", N * (K // group) * 2),
            _ptr(b, "biases", N * (K // group) * 2))


def _gemv(fn, bits, q, s, b, x, y, N, K, M, group, stream):
    if K % group:
        raise MioriError(fn, -2, "K must be a multiple of the group size")
    qp, sp, bp = _qargs(q, s, b, N, K, group, bits)
    od = _out_dtype(y)
    xp = _ptr(x, "x", M * K * 2)
    yp = _ptr(y, "y", M * N * y.element_size())
    if fn.endswith("batched"):
        _lib.call(fn, qp, sp, bp, xp, yp, M, N, K, group, od, _stream(stream))
    else:
        _lib.call(fn, qp, sp, bp, xp, yp, N, K, group, od, _stream(stream))


def gemv4(q, s, b, x, y, N, K, group=64, stream=None):
    """y[N] = dequant4(W)[N][K] . x[K] (src/ops.h:8-10; kernel shaders/ops.metal:6-42)."""
    _gemv("miori_gemv_q4", 4, q, s, b, x, y, N, K, 1, group, stream)


def gemv4_timeline(q, s, b, x, y, N, K, group=64, stream=None):
    """Diagnostic: gemv4 (M = 1, K <= 2048) with four wall-clock stamps per
    wave (entry, loads landed, arithmetic done, stores complete; 100 MHz
    s_memrealtime ticks). Returns an int64 device tensor [waves][4]; y is the
    same as gemv4's. No counterpart in the reference."""
    import ctypes

    if K % group:
        raise MioriError("miori_diag_gemv_q4_timeline", -2, "K must be a multiple of the group size")
    qp, sp, bp = _qargs(q, s, b, N, K, group, 4)
    od = _out_dtype(y)
    xp = _ptr(x, "x", K * 2)
    yp = _ptr(y, "y", N * y.element_size())
    waves = (N + 15) // 16 * 4
    st = torch.zeros((waves, 4), dtype=torch.int64, device=y.device)
    nw = ctypes.c_uint32(0)
    _lib.call("miori_diag_gemv_q4_timeline", qp, sp, bp, xp, yp, N, K, group, od,
              st.data_ptr(), st.numel(), ctypes.byref(nw), _stream(stream))
    assert nw.value == waves
    return st


# The reference's raw-buffer and alternative-lane-map variants compute the
# same product (src/ops.h:105-107, 113-115, 126-128).
gemv4_raw = gemv4
gemv4x4 = gemv4
gemv4x2 = gemv4


def rmsnorm_gemv4(x, norm_w, q, s, b, y, N, K, group=64, eps=1e-5, stream=None):
    """Fused decode step y = W . bf16(rmsnorm(x) * norm_w): the reference's
    rmsnorm -> gemv4 pair (src/engine.cpp:388-393; shaders/ops.metal:86-114,
    6-42) in one launch. x fp32 [K], norm_w bf16 [K]."""
    if K % group:
        raise MioriError("miori_rmsnorm_gemv_q4", -2, "K must be a multiple of the group size")
    if x.dtype != torch.float32 or norm_w.dtype not in (torch.bfloat16, torch.int16):
        raise ValueError("x must be float32 and norm_w bf16")
    qp, sp, bp = _qargs(q, s, b, N, K, group, 4)
    _lib.call("miori_rmsnorm_gemv_q4", _ptr(x, "x", K * 4), _ptr(norm_w, "norm_w", K * 2),
              float(eps), qp, sp, bp, _ptr(y, "y", N * y.element_size()), N, K, group,
              _out_dtype(y), _stream(stream))


def silu_mul_gemv4(gate, up, q, s, b, y, N, K, group=64, stream=None):
    """Fused decode step y = W . bf16(silu(gate) * up): the reference's
    silu_mul -> gemv4 w2 pair (src/engine.cpp:396-398; shaders/ops.metal:129-139,
    6-42) in one launch. gate, up fp32 [K]."""
    if K % group:
        raise MioriError("miori_silu_mul_gemv_q4", -2, "K must be a multiple of the group size")
    if gate.dtype != torch.float32 or up.dtype != torch.float32:
        raise ValueError("gate and up must be float32")
    qp, sp, bp = _qargs(q, s, b, N, K, group, 4)
    _lib.call("miori_silu_mul_gemv_q4", _ptr(gate, "gate", K * 4), _ptr(up, "up", K * 4),
              qp, sp, bp, _ptr(y, "y", N * y.element_size()), N, K, group, _out_dtype(y),
              _stream(stream))


def gemv8(q, s, b, x, y, N, K, group=64, stream=None):
    """8-bit lm_head GEMV (src/ops.h:12-14; kernel shaders/ops.metal:46-82)."""
    _gemv("miori_gemv_q8", 8, q, s, b, x, y, N, K, 1, group, stream)


gemv8_off = gemv8  # src/ops.h:135-138: offsets are tensor views here


def gemv4_b(q, s, b, x, y, N, K, B, group=64, stream=None):
    """Batched 4-bit GEMV over B activation rows, x [B][K] -> y [B][N]
    (src/ops.h:164-166; kernel shaders/batch.metal:145-188, there B <= 4,
    here 1 <= B <= 32)."""
    _gemv("miori_gemv_q4_batched", 4, q, s, b, x, y, N, K, B, group, stream)


def gemv8_b(q, s, b, x, y, N, K, B, group=64, stream=None):
    """Batched 8-bit lm_head (src/ops.h:168-171; shaders/batch.metal:192-236)."""
    _gemv("miori_gemv_q8_batched", 8, q, s, b, x, y, N, K, B, group, stream)


gemv8_b_off = gemv8_b  # src/ops.h:176-179


def gemm_mpp(A, B, C, M, N, K, stream=None):
    """C[M][N] = A[M][K] . B[N][K]^T on MFMA, B the bf16 weight cache written
    by dequant_tile (src/ops.h:94-96; shaders/gemm_mpp.metal:36-54)."""
    ap = _ptr(A, "A", M * K * 2)
    bp = _ptr(B, "B", N * K * 2)
    cp = _ptr(C, "C", M * N * C.element_size())
    _lib.call("miori_gemm_bf16", ap, bp, cp, M, N, K, _out_dtype(C), _stream(stream))


gemm_mpp_off = gemm_mpp  # src/ops.h:101-103
gemm_mpp32 = gemm_mpp    # src/ops.h:207-209 (32-row tile variant of the same product)


def gemm_q4(A, q, s, b, C, M, N, K, group=64, stream=None):
    """Fused 4-bit GEMM: C = A . bf16(dequant4(W))^T with the dequant done
    inside the GEMM (no reference kernel; replaces the reference's
    dequant_tile + gemm_mpp pair, src/engine.cpp:144-146, 508-518)."""
    if K % group:
        raise MioriError("miori_gemm_q4", -2, "K must be a multiple of the group size")
    qp, sp, bp = _qargs(q, s, b, N, K, group, 4)
    ap = _ptr(A, "A", M * K * 2)
    cp = _ptr(C, "C", M * N * C.element_size())
    _lib.call("miori_gemm_q4", ap, qp, sp, bp, cp, M, N, K, group, _out_dtype(C),
              _stream(stream))


def linear(A, q, s, b, C, M, N, K, group=64, bf16_cache=None, stream=None):
    """Batch-engine projection C[M][N] = A[M][K] . W^T with the dispatch
    policy of BatchEngine::linear (src/batch.cpp:223-230): the exact 4-bit
    batched GEMV for M <= 32, else the bf16-cache GEMM when a cache
    (row-major [N][K] bf16, from dequant_tile) is given, else the fused 4-bit
    GEMM."""
    if K % group:
        raise MioriError("miori_linear_q4", -2, "K must be a multiple of the group size")
    qp, sp, bp = _qargs(q, s, b, N, K, group, 4)
    ap = _ptr(A, "A", M * K * 2)
    cp = _ptr(C, "C", M * N * C.element_size())
    cache = 0 if bf16_cache is None else _ptr(bf16_cache, "bf16_cache", N * K * 2)
    _lib.call("miori_linear_q4", ap, qp, sp, bp, cache or None, cp, M, N, K, group,
              _out_dtype(C), _stream(stream))


def gemm_naive(A, B, C, M, N, K, lda, ldb, ldc, aoff=0, boff=0, coff=0, stream=None):
    """C[m*ldc + n] = sum_k A[m*lda + k] * B[n*ldb + k] for any shape, bf16
    operands, fp32 C, one sequential fp32 FMA chain per output (src/ops.h:30-32;
    shaders/ops.metal:199-251). aoff / boff / coff are byte offsets into the
    tensors, as the reference's buffer offsets are."""
    if C.dtype != torch.float32:
        raise ValueError("gemm_naive writes float32")
    for name, off, align in (("aoff", aoff, 2), ("boff", boff, 2), ("coff", coff, 4)):
        if off < 0 or off % align:
            raise ValueError(f"{name} must be a non-negative multiple of {align}")
    ap = _ptr(A, "A", aoff + ((M - 1) * lda + K) * 2)
    bp = _ptr(B, "B", boff + ((N - 1) * ldb + K) * 2)
    cp = _ptr(C, "C", coff + ((M - 1) * ldc + N) * 4)
    _lib.call("miori_gemm_naive", ap + aoff, bp + boff, cp + coff, M, N, K, lda, ldb, ldc,
              _stream(stream))


def _dequant(fn, bits, q, s, b, out, N, K, group, stream):
    if K % group:
        raise MioriError(fn, -2, "K must be a multiple of the group size")
    qp, sp, bp = _qargs(q, s, b, N, K, group, bits)
    if out.dtype != torch.bfloat16:
        raise ValueError("dequant output must be bfloat16")
    op = _ptr(out, "out", N * K * 2)
    _lib.call(fn, qp, sp, bp, op, N, K, group, _stream(stream))


def dequant_tile(q, s, b, out, N, K, group=64, stream=None):
    """4-bit -> bf16 weight cache in the layout gemm_mpp reads, row-major
    [N][K] (src/ops.h:90-92; shaders/gemm_mpp.metal:9-34 writes [N/64][K][64])."""
    _dequant("miori_dequant_q4_tile", 4, q, s, b, out, N, K, group, stream)


def dequant4(q, s, b, out, N, K, group=64, stream=None):
    """4-bit -> bf16 row-major (src/ops.h:26-28; shaders/ops.metal:142-166)."""
    _dequant("miori_dequant_q4", 4, q, s, b, out, N, K, group, stream)


def dequant8(q, s, b, out, N, K, group=64, stream=None):
    """8-bit -> bf16 row-major (src/ops.h:203-205; shaders/ops.metal:754-779)."""
    _dequant("miori_dequant_q8", 8, q, s, b, out, N, K, group, stream)


def sync(stream=None):
    """Block until the stream's work is done (Metal::submit(cb, wait=true))."""
    _lib.call("miori_sync", _stream(stream))


# ---------------------------------------------------------------- uploads
def to_device_bits(a, device="cuda") -> torch.Tensor:
    """numpy uint32 / uint16 host array -> device tensor of the same bits
    (uint32 -> int32 storage, uint16 bf16 bits -> torch.bfloat16)."""
    import numpy as np

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(device)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)
    raise TypeError(f"unsupported dtype {a.dtype}")


def bits_of(t: torch.Tensor):
    """Device bf16 / fp32 tensor -> host numpy array of its bits."""
    import numpy as np

    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.numpy()
    raise TypeError(f"unsupported dtype {t.dtype}")


class QuantLinear:
    """Device copy of one quantized weight matrix (q, scales, biases)."""

    def __init__(self, w, device="cuda"):
        self.q = to_device_bits(w.q, device)
        self.s = to_device_bits(w.s, device)
        self.b = to_device_bits(w.b, device)
        self.bits, self.N, self.K, self.G = w.bits, w.N, w.K, w.G

    def gemv(self, x: torch.Tensor, out_dtype=torch.float32, stream=None) -> torch.Tensor:
        """y[M][N] for x [M][K] (M = 1 -> gemv4/gemv8, M > 1 -> batched)."""
        x = x.reshape(-1, self.K)
        M = x.shape[0]
        y = torch.empty((M, self.N), dtype=out_dtype, device=x.device)
        args = (self.q, self.s, self.b, x, y, self.N, self.K)
        if M == 1:
            (gemv4 if self.bits == 4 else gemv8)(*args, group=self.G, stream=stream)
        else:
            (gemv4_b if self.bits == 4 else gemv8_b)(*args, M, group=self.G, stream=stream)
        return y
