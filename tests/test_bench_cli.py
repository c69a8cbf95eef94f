"""bench.py's command line: the one-GPU contract is enforced before any
device work (a request for several GPUs exits with status 2 and says why)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("n", [2, 8])
def test_bench_refuses_more_than_one_gpu(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)],
                       cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert r.stdout == ""  # no JSON line for a refused run
    assert f"--gpus {n} is not supported" in r.stderr and "one GPU" in r.stderr


def test_bench_rejects_unknown_config():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--config", "nope"],
                       cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "invalid choice" in r.stderr
