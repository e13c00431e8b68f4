"""CPU checks of bench.py's command line (no GPU): more than one GPU is
refused with a message and exit status 2 before anything touches a device,
and the option set the driver and the profiling recipes use parses."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2", "--steps", "5", "--warmup", "1")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_help_lists_the_profiling_options():
    r = _run("--help")
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--case", "--clock", "--calib-copy",
                "--headline-only", "--no-cpu", "--quick"):
        assert opt in r.stdout, opt


def test_help_lists_the_diagnostic_option():
    r = _run("--help")
    assert r.returncode == 0 and "--diag-gemv" in r.stdout


def _bench_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_roofline_picks_the_longer_bound():
    b = _bench_module()
    # the headline GEMV: 9,457,664 B and 33.6 MFLOP, HBM-bound
    r = b.roofline(4.0, 9457664, 2.0 * 8192 * 2048)
    assert r["bound"] == "hbm" and r["unit"] == "GB/s"
    assert abs(r["achieved"] - 9457664 / 4e-6 / 1e9) < 0.1
    assert abs(r["frac"] - r["achieved"] / 8000.0) < 1e-4
    # the M=1024 prefill GEMM: 34.36 GFLOP against 37.7 MB, MFMA-bound
    fl = 2.0 * 1024 * 8192 * 2048
    r = b.roofline(40.0, 1024 * 2048 * 2 + 8192 * 2048 * 2 + 1024 * 8192 * 2, fl)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s"
    assert abs(r["achieved"] - fl / 40e-6 / 1e12) < 0.1


def test_floor_is_launch_plus_stream_time():
    b = _bench_module()
    floors = {"empty_launch_us": 2.0, "copy_stream_GB_s": 5000.0}
    row = b.add_floor({"bytes": 10_000_000, "us": 6.0}, floors)
    assert abs(row["floor_us"] - (2.0 + 10_000_000 / 5e12 * 1e6)) < 1e-3   # 4.0 us
    assert abs(row["floor_frac"] - 4.0 / 6.0) < 1e-3
