"""Test configuration: the ``gpu`` marker and shared helpers.

``-m gpu`` tests need an MI355X and the built library; everything else runs
on the CPU.  The repository root is put on ``sys.path`` so ``oracle`` and
``thundersync_amd`` import from the checkout.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
