"""The skinny kernel's hand-placed vmcnt waits, checked on its gfx950
assembly: no register of a pending load is read or reused early (such a read
gives wrong values; a reuse as an address faults the GPU)."""
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
    bad = {k: v for k, v in res.items() if v}
    assert not bad, {k[:80]: v[:3] for k, v in bad.items()}
    # no register spills: a spill is a copy, and copying a register an inline
    # asm load is still filling reads garbage
    names = re.findall(r"\.name:\s+(_Z\S*skinny_kernel\S*)", text)
    scratch = re.findall(r"\.name:\s+(\S+)(?:(?!\.name:).)*?\.private_segment_fixed_size:\s+(\d+)", text, re.S)
    spilled = [n for n, sz in scratch if "skinny_kernel" in n and int(sz) > 0]
    assert names and not spilled, spilled[:5]
