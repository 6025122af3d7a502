"""Shared test setup: import paths, the ``gpu`` marker, and fixtures.

``-m "not gpu"`` runs the oracle, host logic and ABI checks on the CPU;
``-m gpu`` runs the parity tests through libtempest_hip on an MI355X.
"""
import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "tempest.jl_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built libtempest_hip")


@pytest.fixture(scope="session")
def target():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from tempest_hip import HIPTarget
    return HIPTarget()


def announce(*parts):
    """Name the case on stdout before a GPU step, flushed, so a run that ends
    the box still says what it was doing."""
    print("[case]", *parts, flush=True)
