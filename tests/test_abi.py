"""The C-ABI library loads and exports every symbol include/sluice.h declares
(no GPU work is started here)."""

import ctypes
import os
import re

from sluice_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in sorted(os.listdir(inc)):
        if fn.endswith(".h"):
            src = re.sub(r"/\*.*?\*/", "", open(os.path.join(inc, fn)).read(), flags=re.S)
            names |= set(re.findall(r"\b(sluice_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared()
    assert "sluice_route_topk" in names and "sluice_layer_gap" in names
    assert len(names) >= 20


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = _declared()
    for n in names:
        assert hasattr(lib, n), f"{n} not exported by {_lib.LIB_PATH}"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version_and_errors(lib):
    assert lib.sluice_abi_version() == 1
    assert b"exceeds slots" in lib.sluice_strerror(_lib.SLUICE_E_OVERFLOW)
    assert lib.sluice_strerror(0) == b"ok"


def test_invalid_arguments_rejected_without_touching_the_gpu(lib):
    # shape checks run before any HIP call
    assert lib.sluice_route_topk(None, 0, 1, 0, 1, 0, 0, 1.0, None, 1, 1, None, None,
                                 None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_route_topk(None, 0, 1, 64, 17, 0, 0, 1.0, None, 1, 1, None, None,
                                 None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_moe_align(None, 1, 8, None, 64, 0, None, None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_fused_experts_bf16(None, None, None, None, None, None, 1, 2048, 100, 8, 64,
                                         8, 1.0, None, None, 0, None, None, 0, None, None,
                                         None) == _lib.SLUICE_E_INVAL
    # weight rows stream in 64-element (128-byte) segments: H, I % 64 == 0
    for H, I in ((2048, 96), (2080, 128)):
        assert lib.sluice_fused_experts_bf16(None, None, None, None, None, None, 1, H, I, 8, 64,
                                             8, 1.0, None, None, 0, None, None, 0, None, None,
                                             None) == _lib.SLUICE_E_INVAL
        assert lib.sluice_moe_gemm1_bf16(None, None, None, 1, H, I, 8, None,
                                         None) == _lib.SLUICE_E_INVAL
        assert lib.sluice_moe_gemm2_bf16(None, None, None, None, 1, H, I, 8, None,
                                         None) == _lib.SLUICE_E_INVAL
    # more experts than the align kernel stages in LDS: refused before any
    # launch (pointers are aligned stand-ins; nothing may dereference them)
    fake = 1 << 20
    E_big = _lib.MAX_EXPERTS + 1
    assert lib.sluice_moe_align(fake, 1, 8, fake, E_big, 8, fake, None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_fused_experts_bf16(fake, fake, fake, fake, fake, fake, 1, 2048, 1408, 8,
                                         E_big, 8, 1.0, None, None, 0, None, fake, 1 << 30, fake,
                                         None, None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_fused_experts_fp8(fake, fake, fake, fake, fake, 128, 128, fake, fake, fake,
                                        1, 2048, 1408 // 128 * 128, 8, E_big, 8, 1.0, None, None,
                                        None, None, 0, None, fake, 1 << 30, fake,
                                        None, None) == _lib.SLUICE_E_INVAL
    h = ctypes.c_void_p()
    assert lib.sluice_layer_create(64, 64, 0, 0, None, None, ctypes.byref(h)) == _lib.SLUICE_E_INVAL
    assert lib.sluice_layer_create(2048, 64, 8, 4, None, None,
                                   ctypes.byref(h)) == _lib.SLUICE_E_INVAL


def test_shared_experts_argument_checks(lib):
    """Shared-expert weights whose intermediate is not a multiple of I (or
    above 4*I, or missing) are refused before any device work."""
    args = [ctypes.c_void_p(16)] * 6
    for shared_I, w in ((96, 16), (5 * 64, 16), (128, 0)):
        sw = ctypes.c_void_p(w) if w else None
        rc = lib.sluice_fused_experts_bf16(*args, 2, 256, 64, 2, 8, 4, 1.0, sw, sw, shared_I,
                                           None, ctypes.c_void_p(16), 1 << 30,
                                           ctypes.c_void_p(16), None, None)
        assert rc == _lib.SLUICE_E_INVAL


def test_workspace_size_is_monotone(lib):
    a = lib.sluice_fused_experts_workspace(1, 2048, 1408, 6, 0)
    b = lib.sluice_fused_experts_workspace(8, 2048, 1408, 6, 0)
    c = lib.sluice_fused_experts_workspace(8, 2048, 1408, 6, 2816)
    assert 0 < a < b < c
    assert lib.sluice_moe_plan_ints(8, 6) == 4 + 18 * 48 + 48


def test_add_rmsnorm_gate_shapes(lib):
    ok = lib.sluice_dec_add_rmsnorm_gate_ok
    assert ok(16, 2048) and ok(16, 7168) and ok(1, 8192) and not ok(1, 8200)
    assert not ok(17, 2048) and not ok(4, 2044)


def test_linear_split_parts_and_argument_checks(lib):
    parts = lib.sluice_dec_linear_split_parts
    assert parts(8, 2048, 2048) == 4 and parts(1, 2048, 2048) == 4
    assert parts(8, 2048, 4096) == 3 and parts(16, 2048, 8192) == 4
    assert parts(8, 2048, 256) == 1 and parts(8, 2048, 1024) == 2  # >= 8 K chunks per part
    assert parts(17, 2048, 2048) == 0 and parts(8, 2040, 2048) == 0 and parts(8, 2048, 100) == 0
    # rejected before any launch: bad shapes, misalignment, missing output
    import ctypes
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf)
    p16 = (p + 15) & ~15
    assert lib.sluice_dec_linear_split(p16, p16, 17, 2048, 2048, p16, None) != 0
    assert lib.sluice_dec_linear_split(p16, p16, 8, 2040, 2048, p16, None) != 0
    assert lib.sluice_dec_linear_split(p16 + 4, p16, 8, 2048, 2048, p16, None) != 0
    assert lib.sluice_dec_linear_split(p16, p16, 8, 2048, 2048, None, None) != 0


def test_mla_workspace_grows_with_batch_and_heads(lib):
    ws = lib.sluice_dec_mla_workspace
    assert ws(0, 16) == 0 and ws(1, 0) == 0
    assert 0 < ws(1, 16) < ws(8, 16) < ws(16, 16) < ws(16, 32)


def test_gap_launch_and_read_probe_argument_checks(lib):
    """The gap launch refuses a misaligned plan buffer before looking at the
    layer's device state (a host-only layer has none: SLUICE_E_STATE); the
    read probe refuses null or unaligned buffers and launches nothing for
    zero bytes.  No GPU work is started."""
    h = ctypes.c_void_p()
    lof = (ctypes.c_int32 * 16)(*range(16))
    assert lib.sluice_layer_create(16, 16, 8, 4, lof, None, ctypes.byref(h)) == _lib.SLUICE_OK
    try:
        ids = ctypes.c_void_p(1 << 20)  # an aligned stand-in nothing dereferences
        assert lib.sluice_layer_gap_launch(h, ids, 8, None, None, 0, ctypes.c_void_p((1 << 20) + 2),
                                           None) == _lib.SLUICE_E_INVAL
        assert lib.sluice_layer_gap_launch(h, ids, 8, None, None, 0, None,
                                           None) == _lib.SLUICE_E_STATE
        assert lib.sluice_layer_gap_launch(h, None, 8, None, None, 0, None,
                                           None) == _lib.SLUICE_E_INVAL
    finally:
        assert lib.sluice_layer_destroy(h) == _lib.SLUICE_OK
    sink = ctypes.c_void_p(1 << 20)
    assert lib.sluice_read_probe(None, 16, sink, None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_read_probe(ctypes.c_void_p(1 << 20), 24, sink, None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_read_probe(ctypes.c_void_p((1 << 20) + 8), 16, sink,
                                 None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_read_probe(ctypes.c_void_p(1 << 20), 16, None, None) == _lib.SLUICE_E_INVAL
    assert lib.sluice_read_probe(ctypes.c_void_p(1 << 20), 0, sink, None) == _lib.SLUICE_OK
    assert lib.sluice_gap_set_timeout(-1.0) == _lib.SLUICE_E_INVAL
    assert lib.sluice_gap_set_timeout(float("nan")) == _lib.SLUICE_E_INVAL
    assert lib.sluice_gap_set_timeout(0.0) == _lib.SLUICE_OK
    assert lib.sluice_gap_set_pipelined(2) == _lib.SLUICE_E_INVAL
    assert lib.sluice_gap_set_pipelined(-1) == _lib.SLUICE_E_INVAL
    assert lib.sluice_gap_set_pipelined(0) == _lib.SLUICE_OK
    assert lib.sluice_gap_set_pipelined(1) == _lib.SLUICE_OK
