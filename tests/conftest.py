"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` tests run on any CPU host (oracle, host logic, library exports);
``-m gpu`` tests need an MI355X and compare the HIP path with the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "nnunet-mlx_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def lib(device):
    from nnunet_mlx import _native

    return _native.load()
