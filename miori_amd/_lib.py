"""ctypes binding of libmiori_hip.so (include/miori_hip.h).

The library is the only compute path: if it is missing or fails to load,
every op raises. There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MIORI_HIP_LIB", os.path.join(_PKG, "lib", "libmiori_hip.so"))

# Status codes and dtypes of include/miori_hip.h.
MIORI_OK = 0
MIORI_F32 = 0
MIORI_BF16 = 1

# Every symbol the header declares, with its C signature.
_P, _U, _I = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int
SIGNATURES = {
    "miori_abi_version": ([], _I),
    "miori_status_string": ([_I], ctypes.c_char_p),
    "miori_sync": ([_P], _I),
    "miori_gemv_q4": ([_P, _P, _P, _P, _P, _U, _U, _U, _I, _P], _I),
    "miori_gemv_q8": ([_P, _P, _P, _P, _P, _U, _U, _U, _I, _P], _I),
    "miori_gemv_q4_batched": ([_P, _P, _P, _P, _P, _U, _U, _U, _U, _I, _P], _I),
    "miori_gemv_q8_batched": ([_P, _P, _P, _P, _P, _U, _U, _U, _U, _I, _P], _I),
    "miori_gemm_bf16": ([_P, _P, _P, _U, _U, _U, _I, _P], _I),
    "miori_gemm_q4": ([_P, _P, _P, _P, _P, _U, _U, _U, _U, _I, _P], _I),
    "miori_gemm_q4_static": ([_P, _P, _P, _P, _P, _U, _U, _U, _U, _I, _P], _I),
    "miori_linear_q4": ([_P, _P, _P, _P, _P, _P, _U, _U, _U, _U, _I, _P], _I),
    "miori_gemm_naive": ([_P, _P, _P, _U, _U, _U, _U, _U, _U, _P], _I),
    "miori_rmsnorm_gemv_q4": ([_P, _P, ctypes.c_float, _P, _P, _P, _P, _U, _U, _U, _I, _P], _I),
    "miori_silu_mul_gemv_q4": ([_P, _P, _P, _P, _P, _P, _U, _U, _U, _I, _P], _I),
    "miori_dequant_q4_tile": ([_P, _P, _P, _P, _U, _U, _U, _P], _I),
    "miori_dequant_q4": ([_P, _P, _P, _P, _U, _U, _U, _P], _I),
    "miori_dequant_q8": ([_P, _P, _P, _P, _U, _U, _U, _P], _I),
    "miori_diag_clock_sample": ([_P, _U, _U, _P, _P], _I),
    "miori_diag_gemv_q4_timeline": ([_P, _P, _P, _P, _P, _U, _U, _U, _I, _P, _U, _P, _P], _I),
}

_lib = None


class MioriError(RuntimeError):
    """A non-zero status from libmiori_hip (bad shape, alignment, HIP error)."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn}: {msg} (status {status})")
        self.status = status


def load() -> ctypes.CDLL:
    """Load the library (once). Raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libmiori_hip.so not found at {LIB_PATH}; build it with "
                "`python -m miori_amd.build` (there is no fallback path)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            f = getattr(lib, name)
            f.argtypes = args
            f.restype = res
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise MioriError on a non-zero status."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != MIORI_OK:
        raise MioriError(name, st, lib.miori_status_string(st).decode())


def status(name: str, *args) -> int:
    """Call an entry point and return its raw status."""
    return getattr(load(), name)(*args)
