"""ASan/UBSan build of the host code and the CPU oracle (no GPU): the
safetensors reader (miori_amd/host/weights_hip.cpp) on malformed and randomly
mutated inputs, and the oracle (oracle/cpu_ref.c) on small and ragged
shapes. Any out-of-bounds access or undefined behaviour aborts the run."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpp", "test_host_sanitize.cpp")
OUT = os.path.join(ROOT, "tests", "cpp", "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None,
                    reason="needs gcc/g++")
def test_host_code_under_sanitizers(tmp_path):
    os.makedirs(OUT, exist_ok=True)
    obj = os.path.join(OUT, "cpu_ref_san.o")
    exe = os.path.join(OUT, "test_host_sanitize")
    subprocess.run(["gcc", "-O1", "-std=c11", "-ffp-contract=off", *SAN, "-c",
                    os.path.join(ROOT, "oracle", "cpu_ref.c"), "-o", obj], check=True)
    subprocess.run(["g++", "-O1", "-std=c++17", *SAN, "-D__HIP_PLATFORM_AMD__",
                    f"-I{ROCM}/include", SRC,
                    os.path.join(ROOT, "miori_amd", "host", "weights_hip.cpp"),
                    os.path.join(ROOT, "miori_amd", "host", "metal_hip.cpp"), obj,
                    "-o", exe, f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-lm"],
                   check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=300,
                       env=env)
    print(r.stdout[-3000:], r.stderr[-3000:])
    assert r.returncode == 0 and "ALL PASSED" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]
