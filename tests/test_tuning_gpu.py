"""The tuning experiments behind environment switches compute the same
products as the defaults, bit for bit: MIORI_LMH_NWV=12/16 (the persistent
8-bit kernel with twelve or sixteen waves of 16 blocks in flight),
MIORI_SKINNY_XROT=1 (rotated x-tile DMA order in the skinny and persistent
kernels) and MIORI_LMH_XSUM=1 (the persistent kernel's x sums made once per
workgroup by the same MFMAs). None changes any output's arithmetic or its
order: a tile's blocks are folded in k order by one wave whatever the wave
count and depth, the x tile holds the same bytes whatever order its DMAs run
in, and each x sum is the same MFMA on the same fragments.

The switches are read once per process, so each variant runs in a child
process; the parent computes the default products and compares."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from miori_amd import ops
from tests.gpu_util import acts, say, weights

pytestmark = pytest.mark.gpu

# (kind, bits, M, N, K, G): gemv = the exact batched GEMV, q4 = fused GEMM
CASES = [
    ("gemv", 8, 8, 32776, 2048, 64),     # persistent, one m-tile, ragged N
    ("gemv", 8, 16, 40008, 1024, 128),   # persistent, 16 blocks per tile
    ("gemv", 8, 32, 32784, 2048, 64),    # persistent, two m-tiles
    ("gemv", 4, 32, 8192, 2048, 64),     # skinny, x tile in LDS
    ("q4", 4, 24, 4096, 2048, 64),       # fused skinny, x tile in LDS
]

_CHILD = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from tests.test_tuning_gpu import run_cases
np.savez(sys.argv[2], *run_cases(torch.device("cuda:0")))
print("ok")
"""


def run_cases(dev):
    outs = []
    for kind, bits, M, N, K, G in CASES:
        w, lin = weights(N, K, G, bits, seed=M * 7 + N + K, dev=dev)
        _, xd = acts(M, K, seed=M + K, dev=dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if kind == "gemv":
            (ops.gemv4_b if bits == 4 else ops.gemv8_b)(lin.q, lin.s, lin.b, xd, y, N, K, M,
                                                        group=G)
        else:
            ops.gemm_q4(xd, lin.q, lin.s, lin.b, y, M, N, K, group=G)
        torch.cuda.synchronize()
        outs.append(ops.bits_of(y).reshape(M, N))
    return outs


@pytest.mark.parametrize("env", [{"MIORI_LMH_NWV": "12"}, {"MIORI_LMH_NWV": "16"},
                                 {"MIORI_SKINNY_XROT": "1"}, {"MIORI_LMH_XSUM": "1"}])
def test_tuning_switch_is_bit_identical(dev, tmp_path, env):
    say(f"tuning switch {env} (child process)")
    ref = run_cases(dev)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = tmp_path / "variant.npz"
    r = subprocess.run([sys.executable, "-c", _CHILD, root, str(out)], capture_output=True,
                       text=True, timeout=120, env={**os.environ, **env})
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr[-2000:]
    got = np.load(out)
    for i, case in enumerate(CASES):
        np.testing.assert_array_equal(got[f"arr_{i}"], ref[i], err_msg=str(case))
