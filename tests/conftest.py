"""Shared pytest setup: the `gpu` marker, the repo root on sys.path and the product
package (its directory name has a hyphen, so it is imported through importlib)."""
import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG = "trellis-everywhere_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def te_module():
    return importlib.import_module(PKG)


@pytest.fixture(scope="session")
def te():
    return te_module()


@pytest.fixture(scope="session")
def gpu_device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU (run with -m 'not gpu')")
    return torch.device("cuda:0")
