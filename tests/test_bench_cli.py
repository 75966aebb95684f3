"""bench.py's command-line contract on the CPU: a run asking for more than one GPU is refused with a
message and a non-zero status before anything touches a device (this build measures one GPU; the
driver's multi-GPU launch must not report a figure it did not measure)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    for n in ("2", "8"):
        r = _run("--gpus", n, "--steps", "1", "--warmup", "0")
        assert r.returncode == 2
        assert r.stdout == ""  # no JSON line
        assert f"--gpus {n}" in r.stderr and "one GPU" in r.stderr


def test_help_lists_the_driver_flags():
    r = _run("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--profile", "--calibrate-copy", "--config"):
        assert flag in r.stdout
