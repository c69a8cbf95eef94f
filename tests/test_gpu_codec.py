"""The decode kernel of coded host stores on the GPU: rows coded on the host
(sluice_codec_encode) and decoded in HBM (sluice_codec_decode) equal the
rows bit for bit -- weight-like rows, rows of mostly escaped exponents,
special values, single and many chunks, and a V2-Lite-sized row of 5.8 M
values (its grid-stride loop runs several rounds)."""

import numpy as np
import pytest
import torch

from test_codec import CHUNK, encode, rows_of

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("kind,n", [("weights", CHUNK), ("weights", 2816 * CHUNK),
                                    ("wide", 5 * CHUNK), ("specials", 64 * CHUNK),
                                    ("extremes", 8 * CHUNK), ("constant", 3 * CHUNK)])
def test_decode_kernel_gives_the_rows_back(kind, n):
    from sluice_amd import _lib

    print(f"codec decode {kind} n={n}", flush=True)
    lib = _lib.load()
    v = rows_of(kind, n, seed=n + 7)
    buf = encode(v)
    coded = torch.from_numpy(np.frombuffer(buf + b"\0" * (-len(buf) % 16), dtype=np.uint8).copy())
    coded = coded.to(DEV)
    out = torch.full((n,), 0x5555, dtype=torch.int16, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.sluice_codec_decode(coded.data_ptr(), n, len(buf), out.data_ptr(), st)
    _lib.check(rc, "sluice_codec_decode")
    got = out.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, v)


def test_decode_rejects_bad_sizes():
    from sluice_amd import _lib

    lib = _lib.load()
    v = rows_of("weights", CHUNK)
    buf = encode(v)
    coded = torch.zeros(len(buf) + 16, dtype=torch.uint8, device=DEV)
    out = torch.zeros(CHUNK, dtype=torch.int16, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.sluice_codec_decode(coded.data_ptr(), CHUNK + 16, len(buf), out.data_ptr(),
                                   st) == _lib.SLUICE_E_INVAL
    assert lib.sluice_codec_decode(coded.data_ptr(), CHUNK, 100, out.data_ptr(),
                                   st) == _lib.SLUICE_E_INVAL
    assert lib.sluice_codec_decode(coded.data_ptr(), CHUNK, len(buf) + 2, out.data_ptr(),
                                   st) == _lib.SLUICE_E_INVAL
