"""bench.py's command-line contract on the CPU: one GPU only. Asked for more, it exits with status 2 and says why, before
it imports torch or touches a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    for n in (2, 8):
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)], capture_output=True,
                           text=True, timeout=120)
        assert r.returncode == 2, (n, r.returncode, r.stderr)
        assert "one MI355X" in r.stderr and f"--gpus {n}" in r.stderr, r.stderr
        assert r.stdout == ""  # no JSON line: nothing was measured


def test_help_lists_the_sections():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--no-cpu", "--no-1b", "--no-c3", "--no-engine", "--no-forward",
                 "--no-batch", "--no-fp"):
        assert flag in r.stdout, flag
