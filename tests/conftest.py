"""pytest configuration: the ``gpu`` marker and import paths.

``-m gpu`` tests run the HIP kernels through the C ABI on a ROCm device and
compare them with the CPU oracle (``oracle/``); ``-m "not gpu"`` tests cover
the oracle against known answers and libraries, the host logic, and that the
kernel library loads and exports its symbols.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    return torch.device("cuda", 0)
