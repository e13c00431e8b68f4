"""Hand-placed load waits, checked on the gfx950 assembly of the kernels that
use them (the skinny kernel's inline-asm buffer loads under vmcnt, the GEMM's
inline-asm LDS fragment reads under lgkmcnt): no register of a pending load
is read or reused early on any control-flow path (such a read gives wrong
values; a reuse as an address faults the GPU)."""
import os
import re
import shutil
import subprocess

import pytest

from tests.asm_check import check_file, check_kernel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "miori_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def test_checker_catches_early_use():
    lines = [(1, "global_load_dwordx4 v[2:5], v[0:1], off"), (2, "v_mov_b32_e32 v6, v3"),
             (3, "s_waitcnt vmcnt(0)"), (4, "v_mov_b32_e32 v7, v4")]
    bad = check_kernel(lines)
    assert [b[0] for b in bad] == [2]
    # in-order completion: vmcnt(1) retires the older of two loads only
    lines = [(1, "global_load_dword v2, v[0:1], off"), (2, "global_load_dword v3, v[0:1], off"),
             (3, "s_waitcnt vmcnt(1)"), (4, "v_add_u32_e32 v4, v2, v2"), (5, "v_add_u32_e32 v5, v3, v3")]
    assert [b[0] for b in check_kernel(lines)] == [5]


def test_checker_follows_control_flow():
    # an LDS read issued before a loop is still pending in the loop body
    lines = [(1, "ds_read_b128 v[2:5], v0"), (2, ".LBB0_1:"), (3, "v_add_u32_e32 v7, v2, v2"),
             (4, "s_waitcnt lgkmcnt(0)"), (5, "s_cbranch_scc1 .LBB0_1"), (6, "s_endpgm")]
    assert [b[0] for b in check_kernel(lines)] == [3]
    # a read issued at the bottom of the loop reaches the top over the back edge
    lines = [(1, ".LBB0_1:"), (2, "v_mov_b32_e32 v3, 0"), (3, "ds_read_b32 v3, v0"),
             (4, "s_cbranch_scc1 .LBB0_1"), (5, "s_waitcnt lgkmcnt(0)"), (6, "s_endpgm")]
    # (the loop also never drains its reads, so the queue overflows lgkmcnt)
    assert [b[0] for b in check_kernel(lines) if not isinstance(b[2], str)] == [2]
    # the compiler's if/else flag idiom: only the path that waited branches
    # to the consumer, so no violation
    lines = [(1, "ds_read_b128 v[2:5], v0"), (2, "s_mov_b64 s[4:5], -1"),
             (3, "s_cbranch_scc0 .LBB0_2"), (4, "s_waitcnt lgkmcnt(0)"), (5, "s_mov_b64 s[4:5], 0"),
             (6, ".LBB0_2:"), (7, "s_andn2_b64 vcc, exec, s[4:5]"), (8, "s_cbranch_vccnz .LBB0_3"),
             (9, "s_endpgm"), (10, ".LBB0_3:"), (11, "v_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[2:5], a[0:15]"),
             (12, "s_endpgm")]
    assert check_kernel(lines) == []
    # the same without the wait on the branching path is caught
    lines[3] = (4, "s_nop 0")
    assert [b[0] for b in check_kernel(lines)] == [11]
    # a pending LDS read whose destination is reused by arithmetic (the
    # compiler does this when the read's result is dead)
    lines = [(1, "ds_read_b128 v[6:9], v0"), (2, "v_add_u32_e32 v6, 16, v16"),
             (3, "global_load_lds_dwordx4 v[6:7], off"), (4, "s_endpgm")]
    assert [b[0] for b in check_kernel(lines)] == [2, 3]


def test_checker_catches_counter_overflow():
    # sixteen LDS reads outstanding: lgkmcnt's 4 bits cannot count them
    lines = [(k + 1, f"ds_read_b32 v{k + 10}, v0") for k in range(16)]
    lines.append((17, "s_waitcnt lgkmcnt(0)"))
    bad = check_kernel(lines)
    assert [(b[0], b[2]) for b in bad] == [(16, "lgkmcnt overflow")]
    # fifteen are fine, and a wait between two batches resets the count
    lines = [(k + 1, f"ds_read_b32 v{k + 10}, v0") for k in range(15)]
    lines += [(16, "s_waitcnt lgkmcnt(4)")]
    lines += [(17 + k, f"ds_read_b32 v{k + 40}, v0") for k in range(11)]
    lines.append((40, "s_waitcnt lgkmcnt(0)"))
    assert check_kernel(lines) == []
    # the overflow is found over a loop's back edge too
    lines = [(1, ".LBB0_1:")] + [(k + 2, f"ds_read_b32 v{k + 10}, v0") for k in range(9)]
    lines += [(20, "s_cbranch_scc1 .LBB0_1"), (21, "s_waitcnt lgkmcnt(0)"), (22, "s_endpgm")]
    assert any(b[2] == "lgkmcnt overflow" for b in check_kernel(lines))
    # LDS writes do not count (the compiler drains runs of them with a full wait)
    lines = [(k + 1, f"ds_write_b32 v0, v{k + 10}") for k in range(32)]
    assert check_kernel(lines + [(40, "s_waitcnt lgkmcnt(0)")]) == []


def _compile(src, out):
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S", "-I", CSRC,
           "-o", str(out), os.path.join(CSRC, src)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


def _spilled(text, name):
    scratch = re.findall(r"\.name:\s+(\S+)(?:(?!\.name:).)*?\.private_segment_fixed_size:\s+(\d+)", text, re.S)
    return [n for n, sz in scratch if name in n and int(sz) > 0]


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_gemm_kernel_waits(tmp_path):
    text = _compile("gemm.hip", tmp_path / "gemm.s")
    res = check_file(text, "gemm_kernel")
    assert len(res) == 19, "expected every gemm_kernel instantiation"
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    assert not _spilled(text, "gemm_kernel")
    # the producer / consumer forms: bf16 (DMA producers) and fused 4-bit
    # (consumers load their codes with inline-asm buffer loads two tiles
    # ahead)
    res = check_file(text, "gemm_pc_kernel")
    assert len(res) == 3, "expected every gemm_pc_kernel instantiation"
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    assert not _spilled(text, "gemm_pc_kernel")
    res = check_file(text, "gemm_w8_kernel")
    assert len(res) == 2, "expected every gemm_w8_kernel instantiation"
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    assert not _spilled(text, "gemm_w8_kernel")
    res = check_file(text, "gemm_pcq_kernel")
    assert len(res) == 9, "expected every gemm_pcq_kernel instantiation"
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    assert not _spilled(text, "gemm_pcq_kernel")


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_skinny_kernel_waits(tmp_path):
    out = tmp_path / "skinny.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S", "-I", CSRC,
           "-o", str(out), os.path.join(CSRC, "skinny.hip")]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text()
    res = check_file(text, "skinny_kernel")
    assert len(res) >= 100, "expected every skinny_kernel instantiation"
    # the four-wave forms of the exact modes (template arguments MODE 0/1,
    # MT, NT = 2 or 4, G, NBW, four waves)
    four = [k for k in res if re.search(r"skinny_kernelILi[01]ELi[12]ELi[24]ELi\d+ELi[1248]ELi4EE", k)]
    assert len(four) >= 36, "expected the four-wave instantiations"
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    # no register spills: a spill is a copy, and copying a register an inline
    # asm load is still filling reads garbage
    names = re.findall(r"\.name:\s+(_Z\S*skinny_kernel\S*)", text)
    scratch = re.findall(r"\.name:\s+(\S+)(?:(?!\.name:).)*?\.private_segment_fixed_size:\s+(\d+)", text, re.S)
    spilled = [n for n, sz in scratch if "skinny_kernel" in n and int(sz) > 0]
    assert names and not spilled, spilled[:5]
    # the persistent 8-bit form (M tiles x group x depth, eight waves; and
    # the twelve- and sixteen-wave and x-sum experiments)
    res = check_file(text, "lmh_kernel")
    assert len(res) == 20, "expected every lmh_kernel instantiation"
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    assert not [n for n, sz in scratch if "lmh_kernel" in n and int(sz) > 0]


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_gemv_kernel_waits(tmp_path):
    """The GEMV kernels use compiler-placed waits, plus one hand-placed full
    wait in the stamped diagnostic build (miori_diag_gemv_q4_timeline): the
    checker finds no early use in any instantiation, the diagnostic one
    included, and nothing spills."""
    text = _compile("gemv.hip", tmp_path / "gemv.s")
    res = check_file(text, "gemv_valu_kernel")
    assert len(res) >= 40, "expected every gemv_valu_kernel instantiation"
    assert any("ELi1EEEv" in k for k in res), "the diagnostic instantiation"
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    assert not _spilled(text, "gemv_valu_kernel")
