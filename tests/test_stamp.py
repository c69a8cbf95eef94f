"""Gap mailbox stamps wrap at a multiple of the record ring, so a ring slot
is reused exactly one ring later, also across the wrap (host-only check of
sluice_amd/csrc/stamp.h, compiled with g++)."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not found")
def test_stamps_wrap_at_a_multiple_of_the_ring(tmp_path):
    exe = tmp_path / "stamp_check"
    src = os.path.join(ROOT, "tests", "native", "stamp_check.cpp")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror",
                    f"-I{os.path.join(ROOT, 'sluice_amd', 'csrc')}", src, "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout
