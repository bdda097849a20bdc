from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for path in (ROOT / "ivonar-inference_amd", ROOT / "oracle", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    import ternary_oracle

    return ternary_oracle.oracle()


@pytest.fixture(scope="session")
def cuda():
    """The ROCm device for GPU tests; the HIP library must be built (no fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device in this environment")
    from ivonar_amd import runtime

    runtime.library()  # raises KernelError when the library is missing
    runtime.initialise(0)
    return torch.device("cuda", 0)


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
