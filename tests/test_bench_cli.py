"""bench.py's command-line contract that needs no GPU: it measures one GPU and
refuses a multi-GPU request with a message and exit status 2 before touching
a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = r.stdout + r.stderr
    assert "single GPU" in msg and "--gpus must be 1" in msg
    # no JSON result line is printed for a refused run
    assert not any(line.startswith("{") for line in r.stdout.splitlines())
