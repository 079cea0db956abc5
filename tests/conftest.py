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


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Worst observed normalised errors per MoE parity check, next to its bar."""
    from tests._helpers import BARS, OBSERVED
    if not OBSERVED:
        return
    terminalreporter.section("observed MoE parity errors vs oracle (worst per check)")
    worst: dict = {}
    for check, test, mx, mean in OBSERVED:
        w = worst.setdefault(check, [0.0, 0.0, 0])
        w[0], w[1], w[2] = max(w[0], mx), max(w[1], mean), w[2] + 1
    for check, (mx, mean, n) in sorted(worst.items()):
        bmax, bmean = BARS[check]
        terminalreporter.write_line(f"{check:14s} n={n:3d}  max {mx:.2e} (bar {bmax:.1e})  "
                                    f"mean {mean:.2e} (bar {bmean:.1e})")


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
