"""The host store codec on the CPU: sluice_codec_encode's output, read back
by an independent numpy decoder written from the format the library states
(sign/mantissa bytes, exponent nibbles: an offset from a base per 2048
values, 14 for exponent 0, 15 for an escape listed per chunk), gives every
input row back bit for bit.  The GPU decode is checked against the same
rows in tests/test_gpu_codec.py."""

import ctypes

import numpy as np
import pytest
import torch

from sluice_amd import _lib

CHUNK = 2048


def encode(v: np.ndarray) -> bytes:
    lib = _lib.load()
    v = np.ascontiguousarray(v, dtype=np.uint16)
    need = ctypes.c_size_t()
    assert lib.sluice_codec_encode(v.ctypes.data, v.size, None, 0, ctypes.byref(need)) == 0
    out = np.zeros(need.value // 4 + 1, dtype=np.uint32)
    got = ctypes.c_size_t()
    assert lib.sluice_codec_encode(v.ctypes.data, v.size, out.ctypes.data, out.nbytes,
                                   ctypes.byref(got)) == 0
    assert got.value == need.value
    return out.tobytes()[:got.value]


def decode(buf: bytes, n: int) -> np.ndarray:
    b = np.frombuffer(buf, dtype=np.uint8)
    nc = n // CHUNK
    sm = b[:n].astype(np.uint32)
    nib = b[n:n + n // 2]
    code = np.empty(n, dtype=np.uint32)
    code[0::2] = nib & 0xF
    code[1::2] = nib >> 4
    base = b[n + n // 2:n + n // 2 + nc].astype(np.uint32)
    at = n + n // 2 + ((nc + 3) & ~3)
    off = np.frombuffer(buf[at:at + 4 * (nc + 1)], dtype=np.uint32)
    esc = np.frombuffer(buf[at + 4 * (nc + 1):], dtype=np.uint32)
    assert off[0] == 0 and off[-1] == esc.size and np.all(np.diff(off.astype(np.int64)) >= 0)
    exp = np.where(code == 14, 0, (np.repeat(base, CHUNK) + code) & 0xFF)
    escaped = np.zeros(n, dtype=bool)
    for c in range(nc):
        ent = esc[off[c]:off[c + 1]]
        pos = (ent >> 8).astype(np.int64)
        assert np.all(np.diff(pos) > 0) and np.all(pos < CHUNK)
        exp[c * CHUNK + pos] = ent & 0xFF
        escaped[c * CHUNK + pos] = True
    # exactly the values coded 15 are listed
    assert np.array_equal(escaped, code == 15)
    return (((sm & 0x80) << 8) | (exp << 7) | (sm & 0x7F)).astype(np.uint16)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()


def rows_of(kind: str, n: int, seed: int = 0) -> np.ndarray:
    g = torch.Generator().manual_seed(seed)
    if kind == "weights":
        return bf16_bits(torch.randn(n, generator=g) * 0.02)
    if kind == "wide":  # exponents spread over the whole range: mostly escapes
        return np.random.default_rng(seed).integers(0, 1 << 16, n, dtype=np.uint16)
    if kind == "specials":
        v = bf16_bits(torch.randn(n, generator=g) * 0.02)
        sp = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x0001, 0x807F, 0x7F7F, 0x0080],
                      dtype=np.uint16)
        idx = np.random.default_rng(seed).choice(n, size=min(n, 300), replace=False)
        v[idx] = sp[np.arange(idx.size) % sp.size]
        return v
    if kind == "constant":
        return np.full(n, 0x3C00, dtype=np.uint16)
    if kind == "extremes":  # windows at the two ends of the exponent range
        v = np.empty(n, dtype=np.uint16)
        half = n // 2
        v[:half] = (np.arange(half) % 15 << 7 | np.arange(half) % 128).astype(np.uint16)
        v[half:] = ((240 + np.arange(n - half) % 15) << 7 | 0x8000 |
                    np.arange(n - half) % 128).astype(np.uint16)
        return v
    raise ValueError(kind)


def test_zeros_and_subnormals_are_not_escapes():
    # exponent 0 has a code of its own: a row with 10% zeros (and a few
    # subnormals of either sign) still codes to 0.75 of its bytes
    v = rows_of("weights", 64 * CHUNK, seed=5)
    rng = np.random.default_rng(5)
    v[rng.random(v.size) < 0.1] = 0
    v[rng.choice(v.size, 200, replace=False)] = np.array([0x0001, 0x8003, 0x007F, 0x8000],
                                                         dtype=np.uint16)[np.arange(200) % 4]
    buf = encode(v)
    assert np.array_equal(decode(buf, v.size), v)
    assert len(buf) / (2 * v.size) < 0.753


@pytest.mark.parametrize("kind,n", [("weights", CHUNK), ("weights", 64 * CHUNK),
                                    ("wide", 3 * CHUNK), ("specials", 8 * CHUNK),
                                    ("constant", 2 * CHUNK), ("extremes", 4 * CHUNK)])
def test_round_trip_is_bit_exact(kind, n):
    v = rows_of(kind, n, seed=n)
    buf = encode(v)
    assert np.array_equal(decode(buf, n), v)


def test_weights_code_to_three_quarters():
    n = 1408 * 2048  # one V2-Lite-shaped w2 row block
    v = rows_of("weights", n, seed=1)
    buf = encode(v)
    frac = len(buf) / (2 * n)
    assert 0.75 < frac < 0.754, frac
    # the base of each chunk covers all but a few values in 10^4
    nc = n // CHUNK
    at = n + n // 2 + ((nc + 3) & ~3)
    n_esc = np.frombuffer(buf[at:at + 4 * (nc + 1)], dtype=np.uint32)[-1]
    assert n_esc < n * 5e-4


def test_base_is_the_densest_window():
    # half the chunk at exponent 100, a third at 113 (in one window of 14
    # binades with 100), the rest at 200: base 100 covers 5/6 of the values
    v = np.empty(CHUNK, dtype=np.uint16)
    v[:1024] = 100 << 7
    v[1024:1024 + 683] = 113 << 7
    v[1024 + 683:] = 200 << 7
    buf = encode(v)
    assert buf[CHUNK + CHUNK // 2] == 100
    assert np.array_equal(decode(buf, CHUNK), v)


def test_bad_arguments():
    lib = _lib.load()
    v = np.zeros(CHUNK + 8, dtype=np.uint16)
    need = ctypes.c_size_t()
    assert lib.sluice_codec_encode(v.ctypes.data, v.size, None, 0,
                                   ctypes.byref(need)) == _lib.SLUICE_E_INVAL
    assert lib.sluice_codec_encode(v.ctypes.data, CHUNK, None, 0, ctypes.byref(need)) == 0
    out = np.zeros(need.value // 4 + 1, dtype=np.uint32)
    assert lib.sluice_codec_encode(v.ctypes.data, CHUNK, out.ctypes.data, need.value - 1,
                                   ctypes.byref(need)) == _lib.SLUICE_E_INVAL
