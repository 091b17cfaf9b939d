import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture
def golden():
    import numpy as np

    def load(name):
        return np.load(ROOT / "tests" / "golden" / name, allow_pickle=False)

    return load


@pytest.fixture(autouse=True)
def _full_precision_references():
    """The fp32 oracle must not run on reduced-precision (xf32) matmuls."""
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    yield
