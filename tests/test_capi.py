"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and rejects bad arguments before touching the device (these
calls return from the argument checks; no kernel is launched)."""
import ctypes
import os
import re

import pytest

from miori_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "miori_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(miori_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), f"missing export {n}"
    assert set(names) == set(_lib.SIGNATURES), "binding table out of sync with the header"


def test_version_and_status_strings():
    lib = _lib.load()
    assert lib.miori_abi_version() == 2
    for st in (0, -1, -2, -3, -4, -5, -6):
        assert lib.miori_status_string(st)
    assert lib.miori_status_string(-99) == b"unknown status"


FAKE = 0x10000  # 16-byte aligned, never dereferenced: checks fail first


@pytest.mark.parametrize("args,want", [
    ((0, FAKE, FAKE, FAKE, FAKE, 64, 256, 64, 0, None), -1),        # null q
    ((FAKE, FAKE, FAKE, FAKE, FAKE, 64, 250, 64, 0, None), -2),     # K % 32
    ((FAKE, FAKE, FAKE, FAKE, FAKE, 64, 256, 48, 0, None), -2),     # group
    ((FAKE, FAKE, FAKE, FAKE, FAKE, 64, 65536, 64, 0, None), -2),   # K too large
    ((FAKE, FAKE, FAKE, FAKE, FAKE, 0, 256, 64, 0, None), -2),      # N = 0
    ((FAKE + 4, FAKE, FAKE, FAKE, FAKE, 64, 256, 64, 0, None), -3), # q misaligned
    ((FAKE, FAKE, FAKE, FAKE, FAKE, 64, 256, 64, 7, None), -4),     # dtype
])
def test_gemv_q4_argument_checks(args, want):
    assert _lib.status("miori_gemv_q4", *args) == want


def test_batched_and_gemm_argument_checks():
    assert _lib.status("miori_gemv_q4_batched", FAKE, FAKE, FAKE, FAKE, FAKE,
                       33, 64, 256, 64, 0, None) == -2          # M > 32
    assert _lib.status("miori_gemv_q8_batched", FAKE, FAKE, FAKE, FAKE, FAKE,
                       0, 64, 256, 64, 0, None) == -2           # M = 0
    assert _lib.status("miori_gemv_q8", FAKE, FAKE, FAKE, FAKE, FAKE,
                       64, 256, 8, 0, None) == -2               # group < 16
    assert _lib.status("miori_gemm_bf16", FAKE, FAKE, FAKE, 16, 64, 100, 0, None) == -2
    assert _lib.status("miori_gemm_bf16", FAKE, FAKE, FAKE, 16, 60, 128, 0, None) == -2
    assert _lib.status("miori_gemm_bf16", FAKE, 0, FAKE, 16, 64, 128, 0, None) == -1
    assert _lib.status("miori_gemm_bf16", FAKE + 2, FAKE, FAKE, 16, 64, 128, 1, None) == -3
    assert _lib.status("miori_gemm_q4", FAKE, FAKE, FAKE, FAKE, FAKE, 16, 64, 128, 16, 0, None) == -2
    assert _lib.status("miori_dequant_q4", FAKE, FAKE, FAKE, FAKE, 64, 100, 64, None) == -2
    assert _lib.status("miori_gemm_naive", 0, FAKE, FAKE, 4, 8, 32, 64, 32, 16, None) == -1
    assert _lib.status("miori_gemm_naive", FAKE, FAKE, FAKE, 4, 8, 32, 16, 32, 16, None) == -2  # lda < K
    assert _lib.status("miori_gemm_naive", FAKE, FAKE, FAKE, 4, 8, 32, 64, 32, 4, None) == -2   # ldc < N
    assert _lib.status("miori_gemm_naive", FAKE + 1, FAKE, FAKE, 4, 8, 32, 64, 32, 16, None) == -3
    assert _lib.status("miori_dequant_q8", FAKE, FAKE, FAKE, 0, 64, 128, 64, None) == -1


def test_clock_sampler_argument_checks():
    khz = ctypes.c_uint32(0)
    st = lambda *a: _lib.status("miori_diag_clock_sample", *a)  # noqa: E731
    assert st(0, 16, 50, ctypes.byref(khz), None) == -1            # null samples
    assert st(FAKE, 16, 50, None, None) == -1                      # null wall_khz
    assert st(FAKE, 0, 50, ctypes.byref(khz), None) == -2          # n = 0
    assert st(FAKE, 16, 0, ctypes.byref(khz), None) == -2          # gap = 0
    assert st(FAKE, (1 << 20) + 1, 1, ctypes.byref(khz), None) == -2   # too many samples
    assert st(FAKE + 4, 16, 50, ctypes.byref(khz), None) == -3     # misaligned


def test_ops_rejects_host_tensors():
    import torch

    from miori_amd import ops

    q = torch.zeros(64, dtype=torch.int32)
    with pytest.raises(ValueError):
        ops.gemv4(q, q, q, q, torch.zeros(4), 4, 64)


def test_gemv_timeline_argument_checks():
    n = ctypes.c_uint32(0)
    st = lambda *a: _lib.status("miori_diag_gemv_q4_timeline", *a)  # noqa: E731
    base = (FAKE, FAKE, FAKE, FAKE, FAKE, 8192, 2048, 64, 1)
    assert st(*base, 0, 1 << 16, ctypes.byref(n), None) == -1         # null stamps
    assert st(*base, FAKE, 1 << 16, None, None) == -1                # null nwaves
    assert st(FAKE, FAKE, FAKE, FAKE, FAKE, 8192, 4096, 64, 1, FAKE, 1 << 16,
              ctypes.byref(n), None) == -2                            # K > 2048
    assert st(*base, FAKE + 4, 1 << 16, ctypes.byref(n), None) == -3  # misaligned
    assert st(*base, FAKE, 100, ctypes.byref(n), None) == -2          # too small
    assert n.value == 2048                                            # 512 workgroups x 4
