"""Test configuration: repo root on sys.path, the `gpu` marker, shared helpers.

Tests marked `gpu` run the product (libtrntensor_hip.so on a gfx950 device)
against the CPU oracle in ``oracle/``; they fail, not skip, when the HIP
runtime is missing. Unmarked tests run on any host.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture
def hip():
    """The HIP dispatch module, asserting that the native path is live."""
    from trntensor_amd.hip import dispatch

    assert dispatch.HAS_HIP, f"HIP path unavailable: {dispatch._UNAVAILABLE_REASON}"
    return dispatch
