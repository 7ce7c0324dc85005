import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: large-shape GPU parity runs")


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is not None:
        import torch

        if not torch.cuda.is_available():
            pytest.skip("no ROCm GPU visible")


@pytest.fixture(scope="session")
def device():
    import torch

    return torch.device("cuda", 0)


def pytest_report_header(config):
    return f"rosellm_amd tests (cwd={os.getcwd()})"
