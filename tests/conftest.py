import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "faquant-public_amd")
for path in (REPO, PKG_ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="session")
def golden_codec():
    return load_golden("hif4_codec.npz")


@pytest.fixture(scope="session")
def golden_hadamard():
    return load_golden("hadamard.npz")


@pytest.fixture(scope="session")
def golden_attention():
    return load_golden("attention.npz")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def dev():
    """The MI355X device; GPU tests skip cleanly where there is none."""
    if not gpu_available():
        pytest.skip("needs a ROCm GPU")
    import torch

    return torch.device("cuda:0")
