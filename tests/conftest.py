"""Shared test setup.

Markers:
  gpu   needs an MI355X (runs the HIP engine through libgdn_amd.so);
  slow  long CPU checks, deselected by default with -m "not slow".
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP engine)")
    config.addinivalue_line("markers", "slow: long CPU check")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def gdn():
    import gateddeltanet_amd as g
    from gateddeltanet_amd import _lib
    _lib.load()
    return g
