"""bench.py's command-line contract where it needs no GPU: a request for more
than one GPU ends with a message and a non-zero status before any device or
library is touched, as do invalid step counts."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused():
    for n in ("2", "8"):
        r = run_bench("--gpus", n)
        assert r.returncode == 2, (r.returncode, r.stderr)
        assert "one GPU only" in r.stderr and f"--gpus {n}" in r.stderr
        assert r.stdout == ""


def test_invalid_step_counts_are_refused():
    for args in (("--steps", "0"), ("--warmup", "-1")):
        r = run_bench(*args)
        assert r.returncode != 0 and "steps must be > 0" in r.stderr, (args, r.returncode, r.stderr)
        assert r.stdout == ""
