"""Shared test setup: the ``gpu`` marker and device/oracle fixtures.

``-m "not gpu"`` runs the oracle pins, host logic and ABI checks (no GPU needed);
``-m gpu`` runs the parity tests of the HIP kernels against the oracle.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built backend")


@pytest.fixture(scope="session")
def gpu():
    """The backend module, with a visible GPU (a gpu-marked test fails loudly without one)."""
    import lucid_amd

    if not lucid_amd.is_available():
        pytest.fail("gpu test run without a visible HIP device")
    return lucid_amd


@pytest.fixture(scope="session")
def O():
    import oracle

    oracle.lib()
    return oracle
