"""Shared pytest configuration.

Tests marked `gpu` run the HIP library on a real MI355X; everything else runs
on the CPU (oracle checks, host logic, C-ABI loading and argument checks).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X and the built liblatent_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """Import the product package on a machine with a GPU; fail loudly if anything is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    import latent_amd

    return latent_amd
