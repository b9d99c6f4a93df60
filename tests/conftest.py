"""Shared pytest configuration.

Markers:
  gpu  -- needs an MI355X (HIP device) and the built libbghip.so; these are
          the parity tests proper and call the HIP path through the C ABI.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires a HIP GPU (MI355X) and the built library")


@pytest.fixture(scope="session")
def bridge():
    """One HIP context for the whole GPU session (tests release what they mint)."""
    from browsergrad_amd.bridge import HipRealizerBridge

    br = HipRealizerBridge(device=int(os.environ.get("BG_DEVICE", "0")))
    yield br
    br.close()


@pytest.fixture
def rng():
    import numpy as np

    return np.random.default_rng(1234)
