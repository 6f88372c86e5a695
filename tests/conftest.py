from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return ROOT / "tests" / "golden"


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def built():
    """The compiled library and module; built in place when a fresh checkout lacks them."""
    import neurova_amd
    from neurova_amd import build as nb

    if not (neurova_amd.library_path().exists() and neurova_amd.extension_path().exists()):
        nb.build()
    return True


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the built extension; fails loudly (not skips) when a GPU is present but the build is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import neurova_amd

    neurova_amd.load_extension()  # raises ImportError when not built
    return torch.device("cuda:0")
