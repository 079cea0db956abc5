import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG_NAME = "knivesysl-diffusion-xe_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def load_pkg():
    return importlib.import_module(PKG_NAME)


def load_mod(name: str):
    return importlib.import_module(f"{PKG_NAME}.{name}")


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU (run with -m gpu on the MI355X)")
    from oracle import oracle_c  # noqa: F401  (builds/loads the C oracle)
    load_pkg()._lib.load()
    return torch.device("cuda:0")
