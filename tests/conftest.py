import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    """Build the oracle and the HIP library only when nothing is built (this
    happens on a fresh CPU checkout; GPU boxes receive the prebuilt .so)."""
    from oracle import build_oracle
    if not os.path.exists(build_oracle.OUT):
        build_oracle.build()
    from jules_amd import build as hip_build
    if not os.path.exists(hip_build.LIB):
        hip_build.build()


_ensure_built()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
