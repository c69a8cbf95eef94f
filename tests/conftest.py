import gzip
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs with -m gpu)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        have_gpu = torch.cuda.is_available()
    except Exception:
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


_SLRU = None


def slru_vectors():
    global _SLRU
    if _SLRU is None:
        with gzip.open(os.path.join(GOLDEN, "slru_vectors.json.gz"), "rt") as f:
            _SLRU = json.load(f)
    return _SLRU


@pytest.fixture(scope="session")
def slru_golden():
    return slru_vectors()


_CLASSIC = None


def classic_vectors():
    global _CLASSIC
    if _CLASSIC is None:
        with gzip.open(os.path.join(GOLDEN, "classic_vectors.json.gz"), "rt") as f:
            _CLASSIC = json.load(f)
    return _CLASSIC


@pytest.fixture(scope="session")
def classic_golden():
    return classic_vectors()


@pytest.fixture(scope="session")
def lib():
    from sluice_amd import _lib

    return _lib.load()
