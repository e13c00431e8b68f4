"""GPU run of the C++ host test (tests/cpp/test_ops_host.cpp): the reference's
src/ops.h signatures (Metal&, encoder, Weights&, Tensor&, MTL::Buffer*) over
libmiori_hip.so, on a synthetic MLX-4bit safetensors file, checked against
the CPU oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_ops_host")


@pytest.mark.gpu
def test_ops_h_host_api(dev, tmp_path):
    assert os.path.exists(BIN), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    print(f"running {BIN}", flush=True)
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=240)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "ALL PASSED" in r.stdout


def test_cpp_test_binary_built():
    """The build step produced the host library and the test binary."""
    assert os.path.exists(os.path.join(ROOT, "miori_amd", "lib", "libmiori_host.so"))
    assert os.path.exists(BIN)
