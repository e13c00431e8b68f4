"""HIP-graph capture of every entry-point family (the benchmark times all of
them as graph replays): each call is made eagerly once (which also sizes the
split-K workspace outside capture), captured into a graph, and the graph is
replayed three times. Between replays the output is cleared and other eager
work runs on the same stream, including an eager split-K product that uses
the same per-device workspace. Every replay must reproduce the eager result
bit for bit."""
import numpy as np
import pytest
import torch

from miori_amd import ops, synth
from tests.gpu_util import acts, say, weights

pytestmark = pytest.mark.gpu


def _case(name, dev):
    """(launch function, output tensor) for one entry point."""
    if name == "gemv4":
        _, lin = weights(8192, 2048, 64, 4, seed=11, dev=dev)
        _, x = acts(1, 2048, seed=12, dev=dev)
        y = torch.empty(8192, dtype=torch.bfloat16, device=dev)
        return (lambda: ops.gemv4(lin.q, lin.s, lin.b, x, y, 8192, 2048)), y
    if name == "gemv8":
        _, lin = weights(4096, 2048, 64, 8, seed=13, dev=dev)
        _, x = acts(1, 2048, seed=14, dev=dev)
        y = torch.empty(4096, dtype=torch.float32, device=dev)
        return (lambda: ops.gemv8(lin.q, lin.s, lin.b, x, y, 4096, 2048)), y
    if name.startswith("gemv4_bk"):
        # K = 8192 at M > 8: the K split folded in the kernel (counters)
        M = int(name.split("_m")[1])
        _, lin = weights(2048, 8192, 64, 4, seed=25 + M, dev=dev)
        _, x = acts(M, 8192, seed=26 + M, dev=dev)
        y = torch.empty((M, 2048), dtype=torch.bfloat16, device=dev)
        return (lambda: ops.gemv4_b(lin.q, lin.s, lin.b, x, y, 2048, 8192, M)), y
    if name.startswith("gemv4_b"):
        M = int(name.split("_m")[1])
        _, lin = weights(2048, 2048, 64, 4, seed=15 + M, dev=dev)
        _, x = acts(M, 2048, seed=16 + M, dev=dev)
        y = torch.empty((M, 2048), dtype=torch.bfloat16, device=dev)
        return (lambda: ops.gemv4_b(lin.q, lin.s, lin.b, x, y, 2048, 2048, M)), y
    if name.startswith("gemv8_b_vocab") or name.startswith("gemv4_b_vocab"):
        # vocabulary-sized N: the four-wave skinny forms (8-bit M <= 8 stages x
        # in LDS) and, 8-bit M > 8, the persistent form
        bits = 8 if name.startswith("gemv8") else 4
        M = int(name.split("_m")[1])
        N, K = 32768, 2048
        _, lin = weights(N, K, 64, bits, seed=40 + M, dev=dev)
        _, x = acts(M, K, seed=41 + M, dev=dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        f = ops.gemv8_b if bits == 8 else ops.gemv4_b
        return (lambda: f(lin.q, lin.s, lin.b, x, y, N, K, M)), y
    if name.startswith("gemm_bf16"):
        M, N, K = {"gemm_bf16_splitk": (256, 2560, 2048), "gemm_bf16_192": (1472, 8192, 2048),
                   "gemm_bf16_256": (2048, 8192, 2048), "gemm_bf16_skinny": (24, 2048, 2048)}[name]
        _, A = acts(M, K, seed=17, dev=dev)
        B = (torch.randn(N, K, device=dev) * 0.05).to(torch.bfloat16)
        C = torch.empty((M, N), dtype=torch.float32, device=dev)
        return (lambda: ops.gemm_mpp(A, B, C, M, N, K)), C
    if name == "gemm_q4":
        M, N, K = 1024, 2048, 2048
        _, lin = weights(N, K, 64, 4, seed=18, dev=dev)
        _, A = acts(M, K, seed=19, dev=dev)
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        return (lambda: ops.gemm_q4(A, lin.q, lin.s, lin.b, C, M, N, K)), C
    if name == "gemm_naive":
        M, N, K = 32, 16, 2048
        _, A = acts(M, K, seed=20, dev=dev)
        B = (torch.randn(N, K, device=dev) * 0.05).to(torch.bfloat16)
        C = torch.empty((M, N), dtype=torch.float32, device=dev)
        return (lambda: ops.gemm_naive(A, B, C, M, N, K, K, K, N)), C
    if name == "rmsnorm_gemv4":
        _, lin = weights(2048, 2048, 64, 4, seed=21, dev=dev)
        x = torch.randn(2048, device=dev)
        nw = (torch.rand(2048, device=dev) + 0.5).to(torch.bfloat16)
        y = torch.empty(2048, dtype=torch.float32, device=dev)
        return (lambda: ops.rmsnorm_gemv4(x, nw, lin.q, lin.s, lin.b, y, 2048, 2048)), y
    if name == "silu_mul_gemv4":
        _, lin = weights(2048, 2048, 64, 4, seed=22, dev=dev)
        g = torch.randn(2048, device=dev)
        u = torch.randn(2048, device=dev)
        y = torch.empty(2048, dtype=torch.float32, device=dev)
        return (lambda: ops.silu_mul_gemv4(g, u, lin.q, lin.s, lin.b, y, 2048, 2048)), y
    if name == "dequant_tile":
        _, lin = weights(2048, 2048, 64, 4, seed=23, dev=dev)
        out = torch.empty((2048, 2048), dtype=torch.bfloat16, device=dev)
        return (lambda: ops.dequant_tile(lin.q, lin.s, lin.b, out, 2048, 2048)), out
    raise KeyError(name)


CASES = ["gemv4", "gemv8", "gemv4_b_m4", "gemv4_b_m8", "gemv4_b_m32", "gemv4_bk_m16", "gemv8_b_vocab_m8",
         "gemv8_b_vocab_m32", "gemv4_b_vocab_m24", "gemm_bf16_splitk",
         "gemm_bf16_192", "gemm_bf16_256", "gemm_bf16_skinny", "gemm_q4", "gemm_naive", "rmsnorm_gemv4",
         "silu_mul_gemv4", "dequant_tile"]


@pytest.mark.parametrize("name", CASES)
def test_graph_replay_matches_eager(dev, name):
    say(f"graph replay {name}")
    fn, out = _case(name, dev)
    # unrelated eager work between replays: a torch product and an eager
    # split-K GEMM sharing the library's workspace
    xa = torch.randn(512, 512, device=dev)
    _, A2 = acts(256, 2048, seed=99, dev=dev)
    B2 = (torch.randn(2560, 2048, device=dev) * 0.05).to(torch.bfloat16)
    C2 = torch.empty((256, 2560), dtype=torch.float32, device=dev)
    ops.gemm_mpp(A2, B2, C2, 256, 2560, 2048)
    fn()
    torch.cuda.synchronize()
    ref = ops.bits_of(out).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    for r in range(3):
        out.zero_()
        _ = xa @ xa
        ops.gemm_mpp(A2, B2, C2, 256, 2560, 2048)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ops.bits_of(out), ref, err_msg=f"{name} replay {r}")


def test_graph_replay_after_workspace_growth(dev):
    """A graph captured with a split-K product keeps the workspace address
    it was captured with. An eager split-K product that needs a larger
    workspace allocates a new one and must leave the old one alive: every
    replay after the growth reproduces the eager result bit for bit."""
    say("graph replay after split-K workspace growth")
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def quant(N, K):
        q = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), dtype=torch.int32, device=dev,
                          generator=gen)
        s = (0.001 + 0.009 * torch.rand(N, K // 64, device=dev, generator=gen)).to(torch.bfloat16)
        b = (-8.0 * s.float()).to(torch.bfloat16)
        return q, s, b

    # M = 32, K = 8192: the batched GEMV splits K four ways (partials 4*M*N*4 B)
    M, K = 32, 8192
    N1, N2 = 2048, 262144            # 1 MiB of partials, then 128 MiB
    q1, s1, b1 = quant(N1, K)
    q2, s2, b2 = quant(N2, K)
    x = (torch.randn(M, K, device=dev, generator=gen)).to(torch.bfloat16)
    y1 = torch.empty((M, N1), dtype=torch.float32, device=dev)
    y2 = torch.empty((M, N2), dtype=torch.bfloat16, device=dev)

    def small():
        ops.gemv4_b(q1, s1, b1, x, y1, N1, K, M)

    small()
    torch.cuda.synchronize()
    ref = ops.bits_of(y1).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        small()
    torch.cuda.synchronize()
    for r in range(3):
        y1.zero_()
        ops.gemv4_b(q2, s2, b2, x, y2, N2, K, M)   # grows the workspace on the first pass
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ops.bits_of(y1), ref, err_msg=f"replay {r} after growth")


_FIRST_CAPTURE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np
import torch
from miori_amd import _lib, ops
from tests.gpu_util import acts, weights
_lib.load()
dev = torch.device("cuda:0")
M, N, K = 32, 32768, 2048
_, lin = weights(N, K, 64, 8, seed=77, dev=dev)
_, x = acts(M, K, seed=78, dev=dev)
y = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    ops.gemv8_b(lin.q, lin.s, lin.b, x, y, N, K, M)
torch.cuda.synchronize()
outs = []
for r in range(2):
    y.zero_()
    g.replay()
    torch.cuda.synchronize()
    outs.append(ops.bits_of(y).copy())
y2 = torch.empty_like(y)
ops.gemv8_b(lin.q, lin.s, lin.b, x, y2, N, K, M)
torch.cuda.synchronize()
ref = ops.bits_of(y2)
for o in outs:
    np.testing.assert_array_equal(o, ref)
print("ok")
"""


def test_graph_capture_first_call_persistent(dev):
    """The persistent 8-bit kernel's first call on a device may be made under
    graph capture (it sets the kernel's dynamic-LDS limit once per device
    then): in a fresh process the captured first call replays twice and
    matches a later eager call bit for bit."""
    import os
    import subprocess
    import sys

    say("graph capture of the first persistent-kernel call (child process)")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CAPTURE, root], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr[-2000:]
