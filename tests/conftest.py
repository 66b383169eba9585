"""Test configuration: the `gpu` marker and the repository root on sys.path."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP library")


def gpu_ready() -> bool:
    try:
        import torch

        if not torch.cuda.is_available():
            return False
        from packboost_amd.backends import _hip

        return _hip.device_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip():
    """The loaded HIP library; a GPU test fails loudly if the library or device is missing."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    from packboost_amd.backends import _hip

    lib = _hip.load()
    assert lib.pb_device_available() == 1, "no gfx950 device"
    return _hip


@pytest.fixture(scope="session")
def oracle_mod():
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as o

    o.lib()
    return o
