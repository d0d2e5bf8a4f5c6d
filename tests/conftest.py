import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(autouse=True)
def deterministic_state() -> None:
    """Every test starts from the same torch and numpy RNG state."""
    torch.manual_seed(0)
    np.random.seed(0)


@pytest.fixture
def device() -> torch.device:
    """The GPU under test. GPU tests fail (never skip) when no GPU is visible."""
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")
