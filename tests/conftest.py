import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "gru-triton_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")
    config.addinivalue_line("markers", "slow: long-running case")


@pytest.fixture(scope="session")
def dev():
    """The GPU under test. GPU tests fail (they do not skip) without one, so a
    box whose HIP runtime is broken cannot pass them silently."""
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("GPU test collected but torch.cuda.is_available() is False")
    import gru_qat_amd

    gru_qat_amd.load_library()
    return torch.device("cuda", 0)
