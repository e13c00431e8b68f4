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
