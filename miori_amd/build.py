"""Build libmiori_hip.so in-tree with hipcc for gfx950.

    python -m miori_amd.build          # compile every source, link the library

Objects go to miori_amd/_build/, the library to miori_amd/lib/libmiori_hip.so
(both git-ignored; the library travels with the source tree).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libmiori_hip.so")
HOST_LIB = os.path.join(LIBDIR, "libmiori_host.so")
HOST_SOURCES = ["metal_hip.cpp", "weights_hip.cpp", "ops_hip.cpp"]
ROOT = os.path.dirname(PKG)
CPP_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_ops_host.cpp")
CPP_TEST_BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_ops_host")
ARCH = os.environ.get("MIORI_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
CXX = os.environ.get("CXX", "g++")
# host-only C++ against the HIP runtime API
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__",
              f"-I{ROCM}/include"]
HOST_LINK = [f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"]

SOURCES = ["gemv.hip", "skinny.hip", "dequant.hip", "gemm.hip", "naive.hip", "diag.hip", "workspace.cpp",
           "capi.cpp", "noalloc.cpp"]

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU ops stay disabled in all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unknown-pragmas",
]


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", path, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return obj


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stdout}{r.stderr}")


def build_host() -> str:
    """libmiori_host.so: the src/ops.h-signature C++ host over the C ABI."""
    objs = []
    for src in HOST_SOURCES:
        obj = os.path.join(OBJ, "host_" + os.path.splitext(src)[0] + ".o")
        _run([CXX, *HOST_FLAGS, "-c", os.path.join(PKG, "host", src), "-o", obj],
             f"compile host/{src}")
        objs.append(obj)
    _run([CXX, "-shared", "-fPIC", "-o", HOST_LIB, *objs, "-L" + LIBDIR, "-lmiori_hip",
          "-Wl,-rpath,$ORIGIN", *HOST_LINK], "link libmiori_host.so")
    return HOST_LIB


def build_cpp_test(oracle_lib: str) -> str:
    """tests/cpp test binary (links the host library and the CPU oracle)."""
    os.makedirs(os.path.dirname(CPP_TEST_BIN), exist_ok=True)
    odir = os.path.dirname(oracle_lib)
    _run([CXX, *HOST_FLAGS, CPP_TEST_SRC, "-o", CPP_TEST_BIN, *HOST_LINK, "-L" + LIBDIR,
          "-lmiori_host", "-lmiori_hip", "-L" + odir, "-lmiori_oracle",
          "-Wl,-rpath," + LIBDIR, "-Wl,-rpath," + odir,
          "-Wl,-rpath,$ORIGIN/../../miori_amd/lib", "-Wl,-rpath,$ORIGIN/../../oracle/_build"],
         "build tests/cpp/test_ops_host")
    return CPP_TEST_BIN


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    build_host()
    if verbose:
        print(f"built {LIB} and {HOST_LIB}")
    return LIB


if __name__ == "__main__":
    build()
