"""The native slot cache (sluice_amd/csrc/slru.h) under AddressSanitizer and
UndefinedBehaviorSanitizer: a host-only driver (tests/native/slru_fuzz.cpp,
built with g++) runs random layer shapes -- full and expert-parallel
ownership, pins, LFU and expert counts -- through random router-split gaps
and classic steps and checks the cache's structural invariants after every
operation (each slot in exactly one of free list / probation / protected /
pinned, the two maps inverse of each other, well-linked segment lists,
protected within its cap, every selected owned expert resident after a gap,
plan slots in range).  Parity of the same code with the reference is pinned
by the golden-vector tests; this one adds memory and UB safety."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _sanitizers_available(tmp_path) -> bool:
    probe = tmp_path / "probe.cpp"
    probe.write_text("int main() { return 0; }\n")
    r = subprocess.run(["g++", *SAN, str(probe), "-o", str(tmp_path / "probe")],
                       capture_output=True)
    return r.returncode == 0


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not found")
def test_slot_cache_under_asan_and_ubsan(tmp_path):
    if not _sanitizers_available(tmp_path):
        pytest.skip("g++ has no ASan/UBSan runtime here")
    exe = tmp_path / "slru_fuzz"
    src = os.path.join(ROOT, "tests", "native", "slru_fuzz.cpp")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Werror", *SAN,
                    f"-I{os.path.join(ROOT, 'sluice_amd', 'csrc')}", src, "-o", str(exe)],
                   check=True)
    # the environment may preload a library ahead of the sanitizer runtime
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), "300", "300"], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.stdout[-2000:], r.stderr[-4000:])
