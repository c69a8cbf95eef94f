"""Build libsluice_hip.so in-tree with hipcc for gfx950.

    python -m sluice_amd.build            # sluice_amd/libsluice_hip.so
    python -m sluice_amd.build --trace    # sluice_amd/libsluice_hip_trace.so

Each HIP source compiles to an object in parallel, then one link step makes
``sluice_amd/libsluice_hip.so``.  The library links against the HIP and HSA
runtimes that torch ships (same sonames as /opt/rocm's), with an rpath to
them, so torch and the library always share one runtime of each (load torch
first).
"""

from __future__ import annotations

import os
import re
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
# The decode kernel of coded host stores: a code object of its own, beside
# the libraries, which load it with the HSA loader (csrc/codec.hip).
DECODE_SOURCE = "codec_kernel.hip"
OUT_DECODE = os.path.join(HERE, "codec_decode.hsaco")
BUILD_DIR = os.path.join(ROOT, "_build")

SOURCES = ["routing.hip", "gap.hip", "moe.hip", "decoder.hip", "probe.hip", "codec.hip"]
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


RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"


def _run(cmd: list[str]) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    noise = ("is not a recognized feature for this target", RESOURCE_REMARKS)
    for line in (r.stdout + r.stderr).splitlines():
        if line.strip() and not any(n in line for n in noise) and not line.lstrip().startswith(
                ("|", "^")) and not re.match(r"^\s*\d+ \|", line):
            print(line, file=sys.stderr)
    return r.stdout + r.stderr


# Room the split launch of the expert product must leave per SIMD.  Its
# pending workgroups wait for slots while the copies that fill them run.  The
# gap's copies go to the SDMA engines, but a host-to-device copy that runs as
# a kernel (a HIP-stream copy of small host rows, or any copy with SDMA
# switched off in the runtime) is one 512-thread workgroup (two waves per
# SIMD) allocating 16 VGPRs per lane (the rocprofv3 kernel trace of
# __amd_rocclr_copyBuffer on MI355X).  If the split launch's waves filled the
# 512-VGPR file of every SIMD, such a copy could not start while they wait
# and the waits would run to their bound.
VGPR_FILE = 512
COPY_KERNEL_VGPRS_PER_SIMD = 2 * 16
WAITING_KERNELS = ("moe_gemm2_split_kernel",)
# The gap server's decode of a coded expert (csrc/codec_kernel.hip) runs while the
# split launch's pending workgroups wait for it: one 256-thread workgroup
# (one wave per SIMD) must fit beside their waves.  Coded stores hold bf16
# rows, and a layer's product waits for every expert its gap decodes, so the
# decodes only ever need room beside the bf16 split launch.
DECODE_KERNEL = "sluice_codec_decode_kernel"
DECODE_WAVES_PER_SIMD = 1
DECODE_BESIDE = ("moe_gemm2_split_kernelILb0E",)


def kernel_resources(remarks: str) -> dict[str, dict[str, int]]:
    """{mangled kernel name: {"VGPRs", "AGPRs", "Occupancy"}} from hipcc's
    kernel-resource-usage remarks."""
    out: dict[str, dict[str, int]] = {}
    cur = None
    for line in remarks.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+(VGPRs|AGPRs|Occupancy \[waves/SIMD\]): (\d+)", line)
        if m and cur is not None:
            cur[m.group(1).split()[0]] = int(m.group(2))
    return out


def vgpr_alloc(vgprs: int, agprs: int) -> int:
    """VGPRs a wave holds in gfx950's unified register file: the arch VGPRs
    rounded up to 4, the AGPRs after them, the total in granules of 8."""
    return -(-(-(-vgprs // 4) * 4 + agprs) // 8) * 8


def check_wait_room(remarks: str) -> list[str]:
    """Names of waiting kernels whose waves, at their occupancy, leave less
    than the copy kernel's VGPRs per SIMD free (empty: all fit)."""
    bad = []
    for name, r in kernel_resources(remarks).items():
        if not any(k in name for k in WAITING_KERNELS):
            continue
        used = r["Occupancy"] * vgpr_alloc(r["VGPRs"], r["AGPRs"])
        if VGPR_FILE - used < COPY_KERNEL_VGPRS_PER_SIMD:
            bad.append(f"{name}: {r['Occupancy']} waves x {vgpr_alloc(r['VGPRs'], r['AGPRs'])} "
                       f"VGPRs leave {VGPR_FILE - used} of {COPY_KERNEL_VGPRS_PER_SIMD} free")
    return bad


def check_decode_room(moe_remarks: str, codec_remarks: str) -> list[str]:
    """Waiting bf16 kernels whose waves, at their occupancy, leave less than
    the decode kernel's VGPRs per SIMD free (empty: it fits beside all)."""
    dec = [r for n, r in kernel_resources(codec_remarks).items() if DECODE_KERNEL in n]
    if not dec:
        return [f"{DECODE_KERNEL}: no resource remarks"]
    need = DECODE_WAVES_PER_SIMD * max(vgpr_alloc(r["VGPRs"], r["AGPRs"]) for r in dec)
    bad = []
    for name, r in kernel_resources(moe_remarks).items():
        if not any(k in name for k in DECODE_BESIDE):
            continue
        free = VGPR_FILE - r["Occupancy"] * vgpr_alloc(r["VGPRs"], r["AGPRs"])
        if free < need:
            bad.append(f"{name}: leaves {free} VGPRs per SIMD, the decode needs {need}")
    return bad


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
        cmds.append([hipcc, *HIPCC_FLAGS, *(["-DSLUICE_TRACE"] if trace else []),
                     *([RESOURCE_REMARKS] if src == "moe.hip" else []), "-c",
                     os.path.join(CSRC, src), "-o", obj])
    dec_tmp = os.path.join(bdir, "codec_decode.hsaco")
    cmds.append([hipcc, *HIPCC_FLAGS, "--cuda-device-only", "--no-gpu-bundle-output",
                 RESOURCE_REMARKS, "-c", os.path.join(CSRC, DECODE_SOURCE), "-o", dec_tmp])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        logs = [fut.result() for fut in [ex.submit(_run, c) for c in cmds]]
    bad = check_wait_room(logs[SOURCES.index("moe.hip")])
    if bad:
        raise RuntimeError("kernels that wait on streaming slots leave no room for the "
                           "runtime's copy kernel:\n  " + "\n  ".join(bad))
    bad = check_decode_room(logs[SOURCES.index("moe.hip")], logs[-1])
    if bad:
        raise RuntimeError("kernels that wait on streaming slots leave no room for the "
                           "decode of coded experts:\n  " + "\n  ".join(bad))
    # libhsa-runtime64: the gap's row copies go to the SDMA engines directly
    # (csrc/gap.hip), through the same HSA runtime HIP runs on
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs]
    tl = _torch_lib()
    if tl:
        link += [f"-L{tl}", f"-Wl,-rpath,{tl}"]
    tmp = out + ".tmp"
    link += ["-lhsa-runtime64", "-o", tmp]
    _run(link)
    os.replace(tmp, out)
    shutil.copyfile(dec_tmp, OUT_DECODE + ".tmp")
    os.replace(OUT_DECODE + ".tmp", OUT_DECODE)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True, trace="--trace" in sys.argv[1:])
