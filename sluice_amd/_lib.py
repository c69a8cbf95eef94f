"""ctypes binding of libsluice_hip.so (the C ABI declared in include/sluice.h and
include/sluice_decoder.h).

The shared library is built in-tree (``sluice_amd/libsluice_hip.so``) by
``sluice_amd.build``.  There is no fallback: when the library is missing the
product path raises, so a GPU run can never silently compute on the CPU.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
# SLUICE_TRACE=1 loads the gap-timeline build (python -m sluice_amd.build
# --trace; sluice_amd/timeline.py): the same library with trace hooks.
LIB_PATH = os.path.join(_HERE, "libsluice_hip_trace.so" if os.environ.get("SLUICE_TRACE") == "1"
                        else "libsluice_hip.so")

SLUICE_OK = 0
SLUICE_E_INVAL = -1
SLUICE_E_OVERFLOW = -2
SLUICE_E_TIMEOUT = -3
SLUICE_E_NOMEM = -4
SLUICE_E_STATE = -5
SLUICE_E_ABORTED = -6
SLUICE_E_SCRATCH = -7
SLUICE_E_COPY = -8
NOALLOC_SCRATCH_BYTES = 8 << 20  # SLUICE_NOALLOC_SCRATCH_BYTES

MAX_EXPERTS = 1024
MAX_SLOTS = 512
MAX_TOPK = 16
MAX_PAIRS = 4096
BLOCK_M = 16

# Every symbol include/sluice.h declares: name -> (restype, argtypes).
_P = c_void_p
SIGNATURES = {
    "sluice_abi_version": (c_int, []),
    "sluice_strerror": (ctypes.c_char_p, [c_int]),
    "sluice_route_topk": (
        c_int,
        [_P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P, c_int, c_int, _P, _P, _P],
    ),
    "sluice_slot_lookup": (c_int, [_P, c_int, _P, _P, c_int, _P, c_int32, _P]),
    "sluice_map_refresh": (c_int, [_P, c_int, _P, c_int, _P]),
    "sluice_copy_rows": (c_int, [_P, _P, _P, c_int, _P]),
    "sluice_host_alloc": (c_int, [c_size_t, POINTER(c_void_p)]),
    "sluice_host_free": (c_int, [_P]),
    "sluice_fused_experts_workspace": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "sluice_fused_experts_bf16": (
        c_int,
        [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P, _P, c_int,
         _P, _P, c_size_t, _P, _P, _P],
    ),
    "sluice_fused_experts_bf16_noalloc": (
        c_int,
        [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P, _P, c_int,
         _P, _P, _P, _P],
    ),
    "sluice_fused_experts_fp8": (
        c_int,
        [_P, _P, _P, _P, _P, c_int, c_int, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int,
         c_float, _P, _P, _P, _P, c_int, _P, _P, c_size_t, _P, _P, _P],
    ),
    "sluice_moe_plan_ints": (c_size_t, [c_int, c_int]),
    "sluice_read_probe": (c_int, [_P, c_size_t, _P, _P]),
    "sluice_moe_align": (c_int, [_P, c_int, c_int, _P, c_int, c_int, _P, _P]),
    "sluice_moe_gemm1_bf16": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, _P, _P]),
    "sluice_moe_gemm2_bf16": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, _P]),
    "sluice_moe_gemm1_fp8": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, _P]),
    "sluice_moe_gemm2_fp8": (
        c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, _P]
    ),
    "sluice_moe_combine": (c_int, [_P, _P, c_int, c_int, c_int, c_float, _P, _P, _P]),
    "sluice_layer_create": (c_int, [c_int, c_int, c_int, c_int, _P, _P, POINTER(c_void_p)]),
    "sluice_layer_destroy": (c_int, [_P]),
    "sluice_layer_add_param": (c_int, [_P, _P, _P, c_size_t]),
    "sluice_layer_pulled_params": (c_int, [_P]),
    "sluice_layer_set_staging": (c_int, [_P, c_int]),
    "sluice_layer_stage_counters": (c_int, [_P, _P]),
    "sluice_layer_set_codec": (c_int, [_P, ctypes.c_uint32]),
    "sluice_layer_codec_counters": (c_int, [_P, _P]),
    "sluice_codec_encode": (c_int, [_P, ctypes.c_size_t, _P, ctypes.c_size_t, _P]),
    "sluice_codec_decode": (c_int, [_P, ctypes.c_size_t, ctypes.c_size_t, _P, _P]),
    "sluice_layer_pin": (c_int, [_P, c_int, c_int, POINTER(c_int)]),
    "sluice_layer_gap": (c_int, [_P, _P, c_int, c_int, _P]),
    "sluice_layer_gap_launch": (c_int, [_P, _P, c_int, _P, _P, c_size_t, _P, _P]),
    "sluice_layer_gap_serve": (c_int, [_P, c_int, _P]),
    "sluice_gap_server_create": (c_int, [_P, c_int, c_int, POINTER(c_void_p)]),
    "sluice_gap_server_drain": (c_int, [_P, ctypes.c_double]),
    "sluice_gap_server_error": (c_int, [_P]),
    "sluice_gap_server_destroy": (c_int, [_P]),
    "sluice_gap_abort": (c_int, [c_int]),
    "sluice_gap_set_timeout": (c_int, [c_double]),
    "sluice_gap_set_pipelined": (c_int, [c_int]),
    "sluice_layer_gap_resync": (c_int, [_P]),
    "sluice_layer_unfill": (c_int, [_P, c_int]),
    "sluice_trace_calibrate": (c_int, [c_int, _P, _P]),
    "sluice_trace_read": (c_int, [c_int, _P, POINTER(ctypes.c_uint)]),
    "sluice_trace_reset": (c_int, []),
    "sluice_gap_inject_copy_failure": (c_int, [c_int]),
    "sluice_layer_gap_host": (
        c_int, [_P, _P, c_int, c_int, _P, c_int, POINTER(c_int), POINTER(c_int)]
    ),
    "sluice_layer_state": (
        c_int,
        [_P, _P, _P, _P, POINTER(c_int), _P, POINTER(c_int), _P, POINTER(c_int), _P],
    ),
    "sluice_layer_standing_map": (c_int, [_P, _P]),
    "sluice_layer_classic_plan": (
        c_int, [_P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P, POINTER(c_int)]
    ),
    "sluice_layer_classic_wave": (c_int, [_P, c_int, _P]),
    "sluice_layer_classic_wave_done": (c_int, [_P, c_int, _P]),
    "sluice_layer_classic_host": (
        c_int, [_P, _P, c_int, c_int, c_int, c_int, c_int, c_int, POINTER(c_int)]
    ),
    "sluice_layer_classic_plan_read": (c_int, [_P, _P, c_int, POINTER(c_int), _P]),
    "sluice_layer_set_policy": (c_int, [_P, c_int, c_int]),
    "sluice_layer_policy_state": (c_int, [_P, _P, _P, _P, _P]),
    "sluice_layer_step_stats": (c_int, [_P, _P]),
    # include/sluice_decoder.h
    "sluice_dec_add_rmsnorm": (c_int, [_P, _P, _P, _P, c_int, c_int, c_float, _P]),
    "sluice_dec_silu_mul": (c_int, [_P, _P, c_int, c_int, _P]),
    "sluice_dec_argmax": (c_int, [_P, c_int, c_int, _P, _P]),
    "sluice_dec_linear_workspace": (c_size_t, []),
    "sluice_dec_linear": (c_int, [_P, _P, c_int, c_int, c_int, _P, _P, _P]),
    "sluice_dec_linear_glu": (c_int, [_P, _P, c_int, c_int, c_int, _P, _P, _P]),
    "sluice_dec_add_rmsnorm_gate_ok": (c_int, [c_int, c_int]),
    "sluice_dec_add_rmsnorm_gate": (
        c_int,
        [_P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_float, _P,
         _P],
    ),
    "sluice_dec_linear_split_parts": (c_int, [c_int, c_int, c_int]),
    "sluice_dec_linear_split": (c_int, [_P, _P, c_int, c_int, c_int, _P, _P]),
    "sluice_dec_gate_logits": (
        c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P, _P]
    ),
    "sluice_dec_mla_workspace": (c_size_t, [c_int, c_int]),
    "sluice_dec_mla_decode": (
        c_int,
        [_P, c_int, _P, c_int, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_float, c_float, _P, _P, _P, _P, _P, _P],
    ),
    "sluice_dec_gqa_decode": (
        c_int,
        [_P, _P, c_int, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_float, c_float,
         _P, _P, _P, _P],
    ),
}

_lib = None


class SluiceError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what}: {strerror(code)} (status {code})")


def load() -> ctypes.CDLL:
    """Load the library once (torch first, so its HIP runtime is the one the
    library binds to).  Raises if the library has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (binds libamdhip64 before the library does)

    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libsluice_hip.so not found at {LIB_PATH}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` or "
            "`python -m sluice_amd.build`."
        )
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def strerror(code: int) -> str:
    lib = _lib
    if lib is None:
        return f"status {code}"
    s = lib.sluice_strerror(int(code))
    return s.decode() if s else f"status {code}"


def check(code: int, what: str) -> None:
    if code != SLUICE_OK:
        raise SluiceError(code, what)


def int32_array(values) -> ctypes.Array:
    vals = list(values)
    return (c_int32 * len(vals))(*vals)


__all__ = [
    "LIB_PATH", "SIGNATURES", "SluiceError", "load", "check", "strerror", "int32_array",
    "c_int", "c_int32", "c_int64", "c_size_t", "c_void_p", "POINTER",
]
