"""Build libsluice_hip.so in-tree with hipcc for gfx950.

    python -m sluice_amd.build            # sluice_amd/libsluice_hip.so
    python -m sluice_amd.build --trace    # sluice_amd/libsluice_hip_trace.so

Each HIP source compiles to an object in parallel, then one link step makes
``sluice_amd/libsluice_hip.so``.  The library links against the HIP runtime
that torch ships (same soname as /opt/rocm's), with an rpath to it, so torch
and the library always share one runtime.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(HERE, "libsluice_hip.so")
# The gap-timeline build (-DSLUICE_TRACE: csrc/trace.h), loaded instead of the
# default library when SLUICE_TRACE=1 (sluice_amd/timeline.py sets it).
OUT_TRACE = os.path.join(HERE, "libsluice_hip_trace.so")
BUILD_DIR = os.path.join(ROOT, "_build")

SOURCES = ["routing.hip", "gap.hip", "moe.hip", "decoder.hip", "probe.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Never emit packed fp32 arithmetic (v_pk_{add,mul,fma}_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _torch_lib() -> str | None:
    try:
        import torch

        d = os.path.join(os.path.dirname(torch.__file__), "lib")
        return d if os.path.exists(os.path.join(d, "libamdhip64.so")) else None
    except Exception:
        return None


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    noise = "is not a recognized feature for this target"
    for line in (r.stdout + r.stderr).splitlines():
        if line.strip() and noise not in line:
            print(line, file=sys.stderr)


def build(verbose: bool = False, trace: bool = False) -> str:
    hipcc = _hipcc()
    bdir = os.path.join(BUILD_DIR, "trace") if trace else BUILD_DIR
    out = OUT_TRACE if trace else OUT
    os.makedirs(bdir, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(bdir, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *(["-DSLUICE_TRACE"] if trace else []), "-c",
                     os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for fut in [ex.submit(_run, c) for c in cmds]:
            fut.result()
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs]
    tl = _torch_lib()
    if tl:
        link += [f"-L{tl}", f"-Wl,-rpath,{tl}"]
    tmp = out + ".tmp"
    link += ["-o", tmp]
    _run(link)
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True, trace="--trace" in sys.argv[1:])
